"""naju_amd -- the Naju gated state-space scan as hand-written HIP kernels for
MI355X (gfx950), behind the reference's scan-backend interface.

    from naju_amd import naju_scan_hip, register
    y = naju_scan_hip(u, f_logit, i_logit, B, C, D_skip)     # [B,T,D]
    register()          # NAJU_SCAN_BACKEND=hip now routes naju.NajuMixer here
"""
from naju_amd.scan import (NajuScanHip, naju_scan, naju_scan_hip, register,
                           resolve_backend)

__all__ = ["NajuScanHip", "naju_scan", "naju_scan_hip", "register", "resolve_backend"]
