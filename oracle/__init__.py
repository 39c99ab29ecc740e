"""CPU oracle (test infrastructure only): a plain-PyTorch restatement of the reference
HdcMamba forward path.  Imported by tests/, __graft_entry__.smoke() and bench.py's
CPU-baseline leg, never by the hdcmamba_amd package."""
from .hdcm_oracle import *  # noqa: F401,F403
