"""helrm_amd -- MI355X-native CKKS backend for the HE-LRM embedding PCMM.

The compute path is libhelrm_hip.so (hand-written HIP for gfx950, built from
helrm_amd/csrc by helrm_amd.build).  `HipLibrary` binds it with the method
names of Orion's Lattigo backend; `orion_host` holds the host-side callers of
the path (hybrid diagonal packing, the block loop + rescale, the output fold
and bias, the HE-LRM selector).
"""
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libhelrm_hip.so")


def library_path():
    """Path of the built library; raises if it has not been built."""
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m helrm_amd.build` "
            "(the HIP backend has no CPU fallback)")
    return LIB_PATH


from .backend import HipLibrary, HipError  # noqa: E402,F401
