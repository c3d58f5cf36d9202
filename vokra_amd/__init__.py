"""vokra_amd — MI355X (gfx950) arm of the Vokra quantized-transformer hot path.

The compute lives in libvokra_hip.so (hand-written HIP for CDNA4 behind the C
ABI in include/vokra_hip.h); ``vokra_amd.hip`` is the Python mirror of the
reference's device-context surface. There is no CPU fallback.
"""
from . import hip  # noqa: F401
