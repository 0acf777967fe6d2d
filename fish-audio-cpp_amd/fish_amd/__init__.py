"""MI355X-native W8A8 linear-layer path for fish-audio-cpp's DualAR transformer.

The compute lives in libfish_w8a8.so (HIP, gfx950) behind the C ABI declared in
include/fish_w8a8.h; this package is the Python front end (ctypes binding,
torch-tensor wrappers, .bin reader/writer, synthetic inputs, build).
"""
from ._lib import FaError, lib  # noqa: F401
from .build import LIB_PATH, build_library  # noqa: F401
