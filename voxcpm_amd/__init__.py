"""voxcpm_amd: an MI355X-native (gfx950) implementation of VoxCPM2's
per-patch DiT hot path -- Q8_0 x bf16 products and the local DiT with its
Euler/CFG sampler -- behind a C ABI (include/voxcpm_amd.h).

`voxcpm_amd.ops` holds the torch-facing entry points; `voxcpm_amd.synth`
the seeded synthetic workloads; `voxcpm_amd.build` the gfx950 build.
"""
from ._lib import LIBRARY, VX_BAD_ARG, VX_HIP_ERROR, VX_OK, VX_UNSUPPORTED, VxError, lib

__all__ = ["LIBRARY", "VX_OK", "VX_UNSUPPORTED", "VX_BAD_ARG", "VX_HIP_ERROR",
           "VxError", "lib"]
