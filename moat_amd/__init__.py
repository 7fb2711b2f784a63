"""moat_amd: MI355X (gfx950) implementation of moat's INT4 superblock path.

``moat_amd.dequant`` mirrors the reference's ``src/dequant.py``;
``moat_amd.engine_dequant`` mirrors ``antigravity-engine/src/dequant.py``.
Both run on the HIP kernels of ``libmoat_int4.so`` and need a GPU.
"""

__version__ = "0.1.0"
