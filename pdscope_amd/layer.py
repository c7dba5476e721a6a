"""One MoE layer on the gfx950 kernels with a preallocated workspace.

``moe_forward`` is the whole GPU layer for experts addressed through a slot
table: route (K1) -> decode GEMV (K4) for T == 1, or pack (K2) -> tile
schedule -> grouped SwiGLU (K3) -> merge (K5) for T > 1.  Nothing is
allocated and nothing is read back to the host, so the call can be captured
in a hipGraph (torch.cuda.CUDAGraph) and replayed.
"""
from __future__ import annotations

import torch

from . import ops

BF16 = torch.bfloat16


class MoEWorkspace:
    """Device buffers for up to ``max_tokens`` tokens of one layer shape."""

    def __init__(self, max_tokens: int, H: int, I: int, E: int, k: int, device, *, route_only: bool = False):
        device = torch.device(device)
        n = max_tokens * k
        i32 = dict(dtype=torch.int32, device=device)
        self.max_tokens, self.H, self.I, self.E, self.k, self.device = max_tokens, H, I, E, k, device
        self.logits = torch.empty((max_tokens, E), dtype=BF16, device=device)
        self.ids = torch.empty((max_tokens, k), **i32)
        self.weights = torch.empty((max_tokens, k), dtype=BF16, device=device)
        self.counts = torch.empty(E, **i32)
        self.offsets = torch.empty(E + 1, **i32)
        self.perm_token = torch.empty(n, **i32)
        self.perm_pos = torch.empty(n, **i32)
        self.row_of = torch.empty(n, **i32)
        self.tile_start = torch.empty(E + 1, **i32)
        self.sel_all = torch.arange(E, **i32)
        rows = 1 if route_only else max(n, 1)
        self.h_ws = torch.empty(rows * I, dtype=BF16, device=device)
        self.y = torch.empty(rows * H, dtype=BF16, device=device)
        self.out = torch.empty((1 if route_only else max_tokens, H), dtype=BF16, device=device)
        self.hist = torch.empty(E, **i32)
        self.route_ws = ops.new_route_workspace(max_tokens, H, E, device)
        self.pack_ws = torch.empty(max(ops.pack_workspace_size(max_tokens, k, E), 4), dtype=torch.uint8,
                                   device=device)

    def views(self, T: int):
        if not 0 < T <= self.max_tokens:
            raise ValueError(f"token count {T} outside workspace capacity {self.max_tokens}")
        n = T * self.k
        packed = ops.Packed(self.counts, self.offsets, self.perm_token[:n], self.perm_pos[:n], self.row_of[:n])
        return self.logits[:T], self.ids[:T], self.weights[:T], packed


def route(x, gate, ws: MoEWorkspace, *, normalize=True, bias=None):
    logits, ids, weights, _ = ws.views(x.shape[0])
    ops.route_topk(x, gate, ws.k, normalize, bias=bias, out=(logits, ids, weights), workspace=ws.route_ws)
    return logits, ids, weights


def experts_resident(x, ids, weights, slots, ws: MoEWorkspace, out=None, *, block_m=None):
    """K4 (T == 1) or K2+K3+K5 (T > 1) over experts that are all addressable in `slots`."""
    T = x.shape[0]
    H, I, E, k = ws.H, ws.I, ws.E, ws.k
    out = ws.out[:T] if out is None else out
    if T == 1:
        ops.swiglu_decode(x, ids, weights, slots, H, I, ws.h_ws, out)
        return out
    _, _, _, packed = ws.views(T)
    ops.pack(ids, E, out=packed, workspace=ws.pack_ws)
    bm = block_m or ops.grouped_block_m((T * k) // E)
    ops.schedule(packed.counts, ws.sel_all, bm, out=ws.tile_start)
    max_tiles = (T * k + bm - 1) // bm + E
    ops.swiglu_grouped(x, packed.perm_token, packed.offsets, ws.sel_all, ws.tile_start, max_tiles, bm, slots, H, I,
                       ws.h_ws, ws.y)
    ops.merge(ws.y, packed.row_of, weights, out)
    return out


def moe_forward(x, gate, slots, ws: MoEWorkspace, *, normalize=True, bias=None, block_m=None, fused_decode=True):
    """Full layer: returns (out [T,H] bf16, logits, ids int32 [T,k], weights bf16 [T,k]).

    T == 1 runs the single-launch decode kernel (K4f) when the shape and the
    device allow it (fused_decode), else route (K1) + decode GEMV (K4).
    """
    T = x.shape[0]
    if (T == 1 and fused_decode and ws.k <= 8
            and ops.decode_layer_supported(ws.H, ws.I, ws.E, ws.k, x.device)):
        logits, ids, weights, _ = ws.views(1)
        out = ws.out[:1]
        ops.decode_layer(x, gate, slots, ws.I, ws.k, normalize, bias=bias, out=out, logits=logits, ids=ids,
                         weights=weights, h_ws=ws.h_ws)
        return out, logits, ids, weights
    logits, ids, weights = route(x, gate, ws, normalize=normalize, bias=bias)
    out = experts_resident(x, ids, weights, slots, ws, block_m=block_m)
    return out, logits, ids, weights
