"""MI355X (gfx950) BF16 BSHD D=128 attention forward behind the fav4_bshd C ABI.

The product is ``build/libfav4_bshd.so`` (C ABI in ``include/fav4_bshd.h``);
this package holds its HIP sources (``csrc/``) and the ctypes binding.
"""
from .fav4_bshd import (Args, PagedArgs, Runner, Strides, VarlenArgs, build_library, forward,  # noqa: F401
                        load_library, CEILING_LIB_PATH, LIB_PATH)
