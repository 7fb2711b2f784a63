"""One decoder layer's INT4 projections on MI355X, launched as four GEMMs (the
SwiGLU activation inside the gate/up launch) that a HIP graph can hold.

The projection half of ``antigravity-engine/src/transformer_engine.mm:564-730``
(``forwardLayer``): Q, K and V from the normed hidden state (:582-591), O
from the attention output (:664), gate and up from the post-attention normed
state, ``silu(gate) * up`` (:694-713) and down (:716).  The norms, RoPE, KV
cache, attention and residuals between them are the caller's: they sit
between :meth:`LayerProjections.attention_inputs`, :meth:`output_projection`
and :meth:`mlp`, which enqueue on the current stream, so a caller can capture
its own kernels and these in one graph.  :meth:`capture` records the
projections alone (QKV, O, gate/up + SwiGLU, down) in one graph.

Weights are stored as four matrices instead of seven: ``[W_q | W_k | W_v]``
(hidden x (q_dim + 2 kv_dim)), ``W_o``, ``[W_gate | W_up]`` (hidden x 2
intermediate) and ``W_down``, each one stream of 144-byte records.  In strip
order the stream of a column-concatenated matrix is the concatenation of
its parts' streams (strips are column ranges, stored in column order), so
Q/K/V are one launch.  Gate and up are one launch with the activation: their
strips interleaved (gate strip c, then up strip c), every workgroup holding
whole gate/up pairs and writing fp16 h = silu(gate) * up for their columns
(``moat_int4_gemm_strips_swiglu``), which down reads.  A matrix that strip
order cannot hold (K below 2048) stays in row order, concatenated the same
way through strip order on the device; there gate|up is one launch with an
fp32 output and the SwiGLU kernel makes h from its two halves.

All buffers (inputs, outputs, one GEMM workspace) are allocated once, for
``max_batch`` rows, so that every launch of a call with ``n <= max_batch``
rows has fixed addresses.
"""

from __future__ import annotations

import ctypes
from typing import Any, Dict, Mapping, Tuple

import torch

from . import _device as D
from . import _lib
from .dequant import MAX_BATCH_PER_CALL, SUPERBLOCK_BYTES, SUPERBLOCK_ELEMS, _blob_to_device, records_to_strips, \
    strips_to_records
from .loader import strip_layout_ok

NAMES = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")

__all__ = ["LayerProjections", "NAMES"]


def _weight(entry: Any) -> Tuple[Any, int, int, str]:
    """(records, K, M, layout) from a loader layer dict (``superblocks``,
    ``original_shape``, ``layout``) or a ``(records, K, M)`` tuple of row-order
    records."""
    if isinstance(entry, Mapping):
        shape = entry["original_shape"]
        if len(shape) != 2:
            raise ValueError(f"projection weights are 2-D (K, M), got shape {shape}")
        return entry["superblocks"], int(shape[0]), int(shape[1]), entry.get("layout", "row")
    records, K, M = entry
    return records, int(K), int(M), "row"


def _strips_of(entry: Any) -> torch.Tensor:
    records, K, M, layout = _weight(entry)
    n_sb = K * M // SUPERBLOCK_ELEMS
    blob = _blob_to_device(records, n_sb).reshape(-1)
    return blob if layout == "strip" else records_to_strips(blob, K, M).reshape(-1)


class _Matrix:
    """One GEMM operand: a K x M record stream in strip or row order."""

    def __init__(self, parts, K: int, M: int) -> None:
        self.K, self.M = K, M
        if any(p % 32 for p in self._part_widths(parts)) or K % 8:
            raise ValueError(f"projection widths must be multiples of 32 and K a multiple of 8 (K={K}, "
                             f"widths {self._part_widths(parts)})")
        strips = torch.cat([_strips_of(p) for p in parts]) if len(parts) > 1 else _strips_of(parts[0])
        self.strip = strip_layout_ok((K, M))
        self.blob = strips if self.strip else strips_to_records(strips, K, M).reshape(-1)
        assert self.blob.numel() == K * M // SUPERBLOCK_ELEMS * SUPERBLOCK_BYTES

    @staticmethod
    def _part_widths(parts):
        return [_weight(p)[2] for p in parts]

    def workspace_bytes(self, n: int) -> int:
        lib = _lib.load()
        opt = _lib.GemmOptions()
        if self.strip:
            size = lib.moat_int4_gemm_strips_workspace_size(n, self.K, self.M, ctypes.byref(opt))
        else:
            size = lib.moat_int4_gemm_ex_workspace_size(n, self.K, self.M, ctypes.byref(opt))
        if size < 0:
            raise ValueError(f"no GEMM plan for N={n} K={self.K} M={self.M}")
        return size

    def launch(self, x: torch.Tensor, y: torch.Tensor, n: int, ws: torch.Tensor, what: str) -> None:
        lib = _lib.load()
        opt = _lib.GemmOptions()
        fn = lib.moat_int4_gemm_strips if self.strip else lib.moat_int4_gemm_ex
        for r0 in range(0, n, MAX_BATCH_PER_CALL):
            rows = min(MAX_BATCH_PER_CALL, n - r0)
            _lib.check(fn(x[r0].data_ptr(), self.blob.data_ptr(), y[r0].data_ptr(), rows, self.K, self.M,
                          ctypes.byref(opt), ws.data_ptr(), ws.numel(), D.stream()), what)


class _GateUp:
    """Gate and up with the activation: in strip order their strips
    interleaved for one ``moat_int4_gemm_strips_swiglu`` launch that writes
    h; otherwise ``[W_gate | W_up]`` (fp32 out) and the SwiGLU kernel."""

    def __init__(self, gate, up, K: int, inter: int) -> None:
        self.K, self.inter = K, inter
        self.fused = strip_layout_ok((K, 2 * inter)) and inter % 32 == 0
        if self.fused:
            g, u = _strips_of(gate), _strips_of(up)
            self.blob = torch.empty(2 * g.numel(), dtype=torch.uint8, device=g.device)
            _lib.check(_lib.load().moat_int4_interleave_strips(g.data_ptr(), u.data_ptr(), K, inter,
                                                               self.blob.data_ptr(), D.stream()),
                       "moat_int4_interleave_strips")
            self.strip = True
        else:
            self.mat = _Matrix([gate, up], K, 2 * inter)
            self.blob, self.strip = self.mat.blob, self.mat.strip

    def workspace_bytes(self, n: int) -> int:
        return 0 if self.fused else self.mat.workspace_bytes(n)

    def launch(self, x: torch.Tensor, gate_up, h: torch.Tensor, n: int, ws: torch.Tensor, what: str) -> None:
        lib = _lib.load()
        if self.fused:
            opt = _lib.GemmOptions()
            for r0 in range(0, n, MAX_BATCH_PER_CALL):
                rows = min(MAX_BATCH_PER_CALL, n - r0)
                _lib.check(lib.moat_int4_gemm_strips_swiglu(x[r0].data_ptr(), self.blob.data_ptr(), h[r0].data_ptr(),
                                                            rows, self.K, self.inter, ctypes.byref(opt), D.stream()),
                           what)
            return
        self.mat.launch(x, gate_up, n, ws, what)
        _lib.check(lib.moat_int4_swiglu_f32(gate_up.data_ptr(), n, self.inter, 2 * self.inter, h.data_ptr(),
                                            D.stream()), what + " (swiglu)")


class LayerProjections:
    """The seven projections of one decoder layer, held on the GPU.

    ``weights`` maps ``q_proj``, ``k_proj``, ``v_proj``, ``o_proj``,
    ``gate_proj``, ``up_proj`` and ``down_proj`` (the reference's layer
    weight names, ``transformer_engine.mm:573-716``) to loader layer dicts
    (:meth:`moat_amd.loader.ModelWeightLoader.load_and_repack_layer`, any
    layout) or to ``(records, K, M)`` tuples of row-order records, with K x
    M = in x out: Q hidden x q_dim, K and V hidden x kv_dim, O q_dim x
    hidden, gate and up hidden x intermediate, down intermediate x hidden.
    Every width is a multiple of 32.

    Buffers (fixed addresses, ``max_batch`` rows; a call uses the first n):
    inputs ``x`` (hidden state, fp16), ``attn`` (attention output, fp16),
    ``x_mlp`` (post-attention normed state, fp16); outputs ``qkv`` (fp32, Q
    then K then V per row, also as the views ``q``, ``k``, ``v``), ``o``
    (fp32), ``h`` (fp16 ``silu(gate) * up``), ``down`` (fp32), and, where
    gate and up are not fused with the activation (row order), ``gate_up``
    (fp32, gate then up per row; else None)."""

    def __init__(self, weights: Mapping[str, Any], max_batch: int = 32) -> None:
        missing = [n for n in NAMES if n not in weights]
        if missing:
            raise KeyError(f"missing projection weights: {missing}")
        if max_batch < 1:
            raise ValueError("max_batch must be >= 1")
        dev = D.require_gpu()
        _lib.load()
        shapes = {n: _weight(weights[n])[1:3] for n in NAMES}
        H, q_dim = shapes["q_proj"]
        kv_dim = shapes["k_proj"][1]
        inter = shapes["gate_proj"][1]
        want = {"q_proj": (H, q_dim), "k_proj": (H, kv_dim), "v_proj": (H, kv_dim), "o_proj": (q_dim, H),
                "gate_proj": (H, inter), "up_proj": (H, inter), "down_proj": (inter, H)}
        for n in NAMES:
            if shapes[n] != want[n]:
                raise ValueError(f"{n}: shape {shapes[n]} does not fit hidden={H} q_dim={q_dim} "
                                 f"kv_dim={kv_dim} intermediate={inter} (expected {want[n]})")
        self.hidden, self.q_dim, self.kv_dim, self.intermediate = H, q_dim, kv_dim, inter
        self.max_batch = int(max_batch)
        self.qkv_w = _Matrix([weights["q_proj"], weights["k_proj"], weights["v_proj"]], H, q_dim + 2 * kv_dim)
        self.o_w = _Matrix([weights["o_proj"]], q_dim, H)
        self.gate_up_w = _GateUp(weights["gate_proj"], weights["up_proj"], H, inter)
        self.down_w = _Matrix([weights["down_proj"]], inter, H)
        mats = (self.qkv_w, self.o_w, self.gate_up_w, self.down_w)
        ws_bytes = max(m.workspace_bytes(n) for m in mats for n in range(1, min(self.max_batch, MAX_BATCH_PER_CALL) + 1))
        ws_bytes = max(ws_bytes, 256)
        self.workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        _lib.check(_lib.load().moat_int4_workspace_clear(self.workspace.data_ptr(), ws_bytes, D.stream()),
                   "moat_int4_workspace_clear")
        B = self.max_batch
        f16, f32 = torch.float16, torch.float32
        self.x = torch.zeros((B, H), dtype=f16, device=dev)
        self.attn = torch.zeros((B, q_dim), dtype=f16, device=dev)
        self.x_mlp = torch.zeros((B, H), dtype=f16, device=dev)
        self.qkv = torch.empty((B, q_dim + 2 * kv_dim), dtype=f32, device=dev)
        self.q = self.qkv[:, :q_dim]
        self.k = self.qkv[:, q_dim:q_dim + kv_dim]
        self.v = self.qkv[:, q_dim + kv_dim:]
        self.o = torch.empty((B, H), dtype=f32, device=dev)
        self.gate_up = None if self.gate_up_w.fused else torch.empty((B, 2 * inter), dtype=f32, device=dev)
        self.h = torch.empty((B, inter), dtype=f16, device=dev)
        self.down = torch.empty((B, H), dtype=f32, device=dev)
        self._graphs: Dict[int, torch.cuda.CUDAGraph] = {}

    @property
    def weight_bytes(self) -> int:
        return sum(m.blob.numel() for m in (self.qkv_w, self.o_w, self.gate_up_w, self.down_w))

    @property
    def layouts(self) -> Dict[str, str]:
        return {name: ("strip" if m.strip else "row") for name, m in
                (("qkv", self.qkv_w), ("o", self.o_w), ("gate_up", self.gate_up_w), ("down", self.down_w))}

    def _rows(self, n: int) -> int:
        n = int(n)
        if not 1 <= n <= self.max_batch:
            raise ValueError(f"n must be in 1..{self.max_batch} (got {n})")
        return n

    def attention_inputs(self, n: int) -> None:
        """Enqueue Q, K, V = x[:n] @ [W_q | W_k | W_v] (one launch) into ``qkv``."""
        n = self._rows(n)
        self.qkv_w.launch(self.x, self.qkv, n, self.workspace, "LayerProjections.qkv")

    def output_projection(self, n: int) -> None:
        """Enqueue o = attn[:n] @ W_o."""
        n = self._rows(n)
        self.o_w.launch(self.attn, self.o, n, self.workspace, "LayerProjections.o")

    def mlp_front(self, n: int) -> None:
        """Enqueue h = fp16(silu(x_mlp[:n] @ W_gate) * (x_mlp[:n] @ W_up)): one
        launch in strip order, else the gate|up launch and the SwiGLU kernel."""
        n = self._rows(n)
        self.gate_up_w.launch(self.x_mlp, self.gate_up, self.h, n, self.workspace, "LayerProjections.gate_up")

    def down_projection(self, n: int) -> None:
        """Enqueue down = h[:n] @ W_down."""
        n = self._rows(n)
        self.down_w.launch(self.h, self.down, n, self.workspace, "LayerProjections.down")

    def mlp(self, n: int) -> None:
        """:meth:`mlp_front` then :meth:`down_projection`."""
        self.mlp_front(n)
        self.down_projection(n)

    def run(self, n: int) -> None:
        """Enqueue every projection of the layer for the first n rows."""
        self.attention_inputs(n)
        self.output_projection(n)
        self.mlp(n)

    def capture(self, n: int) -> torch.cuda.CUDAGraph:
        """A HIP graph of :meth:`run` for n rows (cached per n).  Replaying it
        reads the current contents of ``x``, ``attn`` and ``x_mlp``.  Graphs of
        one layer share its workspace: replay them on one stream at a time."""
        n = self._rows(n)
        g = self._graphs.get(n)
        if g is not None:
            return g
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self.run(n)  # first launches (kernel attributes) outside the capture
        side.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            self.run(n)
        torch.cuda.current_stream().wait_stream(side)
        self._graphs[n] = g
        return g

    def forward(self, x, attn, x_mlp, graph: bool = True) -> Dict[str, torch.Tensor]:
        """Copy the three inputs (each (n, width), any float dtype, rounded
        to fp16) into the layer's buffers and run the projections (the
        captured graph for n rows when ``graph``).  Returns views of the
        outputs' first n rows: ``q``, ``k``, ``v``, ``o``, ``h``, ``down``."""
        xs = [D.to_device(a) for a in (x, attn, x_mlp)]
        n = xs[0].shape[0] if xs[0].dim() == 2 else 1
        for src, dst in zip(xs, (self.x, self.attn, self.x_mlp)):
            src = src.reshape(-1, dst.shape[1])
            if src.shape[0] != n:
                raise ValueError("x, attn and x_mlp need the same number of rows")
            self._rows(n)
            dst[:n].copy_(src)
        if graph:
            self.capture(n).replay()
        else:
            self.run(n)
        return {"q": self.q[:n], "k": self.k[:n], "v": self.v[:n], "o": self.o[:n], "h": self.h[:n],
                "down": self.down[:n]}

    def check(self) -> None:
        """Raise RuntimeError if a hand-off between workgroups in this layer's
        GEMMs ran out of time since the last check (those results were NaN);
        clears the workspace first.  Synchronises the current stream."""
        lib = _lib.load()
        st = ctypes.c_int32(0)
        _lib.check(lib.moat_int4_workspace_status(self.workspace.data_ptr(), self.workspace.numel(),
                                                  ctypes.byref(st), D.stream()), "moat_int4_workspace_status")
        if st.value:
            _lib.check(lib.moat_int4_workspace_clear(self.workspace.data_ptr(), self.workspace.numel(), D.stream()),
                       "moat_int4_workspace_clear")
            raise RuntimeError(f"LayerProjections: a hand-off between workgroups ran out of time (status {st.value})")
