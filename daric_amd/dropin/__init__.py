"""Files that drop this package into a DARIC source tree in place of the
reference's CUDA extension and Triton adapter. Each module's docstring names
the path it replaces; it only re-exports daric_amd's implementation."""
