"""adana_amd: MI355X-native ADana-family optimizer step.

``ADana`` (ADana / Dana-MK4) and ``DANA_STAR_MK4`` (Dana-Star / Dana-Star-MK4)
are drop-ins for mlexpos/adana's src/optim/adana.py and
src/optim/dana_star_mk4.py whose step() runs one hand-written gfx950 HIP
multi-tensor kernel (adana_amd/csrc/adana_mta.hip) through the C ABI in
include/adana_mta.h.  ``Manau`` (src/optim/manau.py) runs its Dana-Star-MK4
branch on the same kernel.
"""
from .clip import clip_grad_norm_
from .manau import Manau
from .optim import ADana, DANA_STAR_MK4, DIAG_KEYS
from .schedules import log_optimizer_schedules
from .tau_stats import compute_tau_order_statistics, extract_tau_statistics

__all__ = ["ADana", "DANA_STAR_MK4", "DIAG_KEYS", "Manau", "clip_grad_norm_", "log_optimizer_schedules",
           "compute_tau_order_statistics", "extract_tau_statistics"]
