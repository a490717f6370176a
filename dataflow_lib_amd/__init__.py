"""MI355X-native (gfx950) implementation of dataflow_lib's native op path.

The product is the C ABI in include/*.h, implemented by lib/libdataflow.so
(registry + HIP backend), lib/libdataflow_hip_config.so (launch geometry) and
lib/dataflow_kernels_gfx950.hsaco (hand-written HIP kernels). This package
builds them (build.py) and binds them for Python callers (api.py).
"""
from . import api  # noqa: F401
