"""MI355X-native (gfx950) W4A8 / W8A8 quantized linear for the HC-Zhou/open_rknpu2_lm_infer engine.

libqlinear.so (built from csrc/ by build.py) holds the HIP kernels and the C ABI of
include/qlinear.h.  _lib binds that ABI with ctypes; qlinear is a torch-tensor front
end over it; synth makes the seeded synthetic workloads.
"""
from . import _lib  # noqa: F401

__all__ = ["_lib"]
