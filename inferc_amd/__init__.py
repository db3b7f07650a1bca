"""inferc_amd — MI355X (gfx950) backend for inferc's runtime hot path.

The compute lives in ``libinferc_hip.so`` (hand-written HIP kernels behind the
C-ABI of ``include/inferc_hip.h``). This package is the Python host side over
that ABI: it loads the library, declares every entry point for ``ctypes`` and
wraps them with inferc's operator names (see :mod:`inferc_amd.rt`). There is no
CPU fallback: if the library is missing, importing :mod:`inferc_amd.rt` or
creating a :class:`Context` raises.
"""
from .lib import HipError, load_library, library_path  # noqa: F401

__all__ = ["HipError", "load_library", "library_path"]
