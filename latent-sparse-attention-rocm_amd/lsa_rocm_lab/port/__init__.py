"""The select+read port surface on MI355X (reference src/lsa_rocm_lab/port/__init__.py).

The reference bootstraps an upstream checkout and re-exports its Triton modules
(port/__init__.py:39-56). This package has no upstream or Triton dependency: the
package only locates the HIP library, loaded lazily on the first kernel call.
"""

import pathlib

from lsa_rocm_lab import _abi

ROOT = pathlib.Path(__file__).resolve().parents[3]
HIP_ARCH = "gfx950"
LIBRARY = _abi.LIB_PATH


def library_loaded() -> bool:
    """True once liblsa_rocm.so has been loaded into this process."""
    return _abi._lib is not None


__all__ = ["ROOT", "HIP_ARCH", "LIBRARY", "library_loaded"]
