"""MI355X (gfx950) HIP backend for the Qwen3 decode/prefill path of almostrealism/common.

The compute path is the native library ``common_amd/lib/libar_hip.so`` (C-ABI in
``include/ar_hip.h``); the Python modules here are thin bindings over it:

* ``hardware``  -- context / memory provider / operators (the backend SPI objects)
* ``qwen3``     -- Qwen3 + AutoregressiveModel token loop
* ``config``    -- Qwen3Config and the benchmark configurations
* ``synthetic`` -- seeded synthetic weights and prompts
"""
from .config import Qwen3Config  # noqa: F401
