"""CPU oracle (test infrastructure only; never imported by ``moat_amd``)."""

from .superblock_oracle import *  # noqa: F401,F403
