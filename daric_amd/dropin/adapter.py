"""Copy over daric/adaption/adapter.py in a DARIC tree: the package's
`from .adapter import Adapter` (daric/adaption/__init__.py) and the worker's
Adapter(config.adaption_config) (daric/cache_engine.py:260) then build the
gfx950 Adapter, which reads ProcessLocalConfig.cache_topo as the reference's
does (adapter.py:94, 154, 241, 311).
"""
from daric_amd.adapter import Adapter  # noqa: F401
