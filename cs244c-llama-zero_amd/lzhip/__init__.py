"""Python side of the gfx950 kernel library: ctypes binding (_lib), tensor-level
wrappers (ops) and autograd functions (functional)."""
from . import _lib, ops  # noqa: F401
from ._lib import HipLibraryError, load  # noqa: F401
