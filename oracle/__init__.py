"""CPU oracle (test infrastructure only; never imported by ``moat_amd``)."""

from .superblock_oracle import *  # noqa: F401,F403
from .dense_oracle import dense_exact, dense_gemm_ref, dense_tolerance, fp16_ulp, gemv_ref  # noqa: F401
