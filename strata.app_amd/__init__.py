"""MI355X-native Prefill MoE layer (the reference's strata::metal Prefill MoE coordinators).

The directory name is not a Python identifier; load it with `load_package()` from
`__graft_entry__.py` (registered as module `strata_app_amd`). Submodules:
  moe    — ctypes mirror of the C ABI in include/strata_moe.h (contexts, views, segments,
           coordinators, synthetic inputs)
  layer  — benchmark configurations, seeded inputs and a device workspace for one layer
  gguf_write — writes GGUF model files of routed-expert tensors (synthetic model files)
  build  — builds libstrata_moe.so for gfx950
"""
from . import moe, layer, gguf_write  # noqa: F401
