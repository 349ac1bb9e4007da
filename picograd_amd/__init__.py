"""picograd-amd: MI355X-native backward pass of picograd behind its C ABI.

The product is the C library lib/libpicograd_amd.so (include/picograd/*.h);
this package only builds it (`build`) and binds it for Python callers
(`capi`).  Loading fails loudly when the library is missing.
"""
from .capi import PgLib, load, F32, F16, BF16  # noqa: F401

__all__ = ["PgLib", "load", "F32", "F16", "BF16"]
