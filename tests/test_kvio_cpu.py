"""KVIOContext's host-side limits (CPU only): the staging size setting the
reference reads (DARIC_KV_IPC_STAGING_MB, gpu_kv_io.py:30-34) and the greedy
batching of metas into staging buffers (gpu_kv_io.py:445-462): at most
MAX_BATCH_SIZE metas and staging_bytes per batch, a meta of exactly
staging_bytes accepted and a larger one refused, as the reference accepts
and refuses them."""
import importlib

import pytest

from daric_amd import kv_io


def test_staging_size_setting(monkeypatch):
    monkeypatch.delenv("DARIC_KV_IPC_STAGING_MB", raising=False)
    assert kv_io._staging_bytes_from_env() == 256 << 20
    monkeypatch.setenv("DARIC_KV_IPC_STAGING_MB", "64")
    assert kv_io._staging_bytes_from_env() == 64 << 20
    monkeypatch.setenv("DARIC_KV_IPC_STAGING_MB", "0")
    with pytest.raises(ValueError, match="must be positive"):
        kv_io._staging_bytes_from_env()
    # the module's default follows the setting at import
    monkeypatch.setenv("DARIC_KV_IPC_STAGING_MB", "32")
    try:
        assert importlib.reload(kv_io).DEFAULT_STAGING_BYTES == 32 << 20
    finally:
        monkeypatch.delenv("DARIC_KV_IPC_STAGING_MB")
        importlib.reload(kv_io)


def batches(sizes, cap, max_count=kv_io.KVIOContext.MAX_BATCH_SIZE):
    return list(kv_io.KVIOContext._batches(None, sizes, cap, max_count))


def test_batches_follow_the_reference_limits():
    cap = 1 << 20
    assert batches([cap], cap) == [(0, 1)]                       # a meta of exactly one buffer
    assert batches([cap // 2] * 5, cap) == [(0, 2), (2, 4), (4, 5)]
    assert batches([10] * 9, cap) == [(0, 4), (4, 8), (8, 9)]    # at most 4 metas a batch
    assert batches([cap // 2, cap, 1], cap) == [(0, 1), (1, 2), (2, 3)]
    with pytest.raises(RuntimeError, match="larger than the 1048576-byte staging buffer"):
        batches([1, cap + 1], cap)
