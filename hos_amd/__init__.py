"""hos_amd — MI355X (gfx950) backend for HOS's LoRA fine-tuning path.

The compute lives in libhos_hip.so (hand-written HIP for gfx950 behind the C ABI of
include/hos_hip.h); this package is the host-side mirror of the reference's interfaces.
"""
from .hip_be import Gpu, HosError, bytes_for  # noqa: F401
