"""One MoE layer on the gfx950 kernels with a preallocated workspace.

``moe_forward`` is the whole GPU layer for experts addressed through a slot
table: route (K1) -> decode GEMV (K4) for T == 1, or pack (K2) -> balanced tile
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

    def __init__(self, max_tokens: int, H: int, I: int, E: int, k: int, device, *, route_only: bool = False,
                 shared_I: int | None = None):
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
        self.sel_order = torch.empty(E, **i32)  # balanced expert order of the grouped launch
        self.tile_start_down = torch.empty(E + 1, **i32)  # the down launch's own tiling (down_block_m)
        self.sel_all = torch.arange(E, **i32)
        rows = 1 if route_only else max(n, 1)
        self.h_ws = torch.empty(rows * I, dtype=BF16, device=device)
        self.y = torch.empty(rows * H, dtype=BF16, device=device)
        self.out = torch.empty((1 if route_only else max_tokens, H), dtype=BF16, device=device)
        self.hist = torch.empty(E, **i32)
        self.route_ws = ops.new_route_workspace(max_tokens, H, E, device)
        self.pack_ws = torch.empty(max(ops.pack_workspace_size(max_tokens, k, E), 4), dtype=torch.uint8,
                                   device=device)
        # always-on shared experts (one fused MLP of intermediate shared_I over every token)
        self.shared_I = shared_I
        if shared_I:
            self.h_shared = torch.empty(max_tokens * shared_I, dtype=BF16, device=device)
            self.y_shared = torch.empty((max_tokens, H), dtype=BF16, device=device)
            self.shared_rows = torch.arange(max_tokens, **i32)
            self.shared_offsets = torch.zeros(2, **i32)
            self.shared_tiles = torch.zeros(2, **i32)
            self.shared_sel = torch.zeros(1, **i32)
            self._shared_key = None    # (T, row tile) the two tables above hold
            self._side = None

    def side_stream(self):
        """A second stream on the workspace's device (default priority) for
        the shared experts, which run beside the routed ones."""
        if self._side is None:
            self._side = torch.cuda.Stream(device=self.device)
        return self._side

    def pregathered(self, n: int) -> torch.Tensor:
        """[n, H] bf16 buffer for activation rows gathered into grouped order."""
        buf = getattr(self, "_xg", None)
        if buf is None or buf.shape[0] < n:
            buf = torch.empty((max(n, self.max_tokens * self.k), self.H), dtype=BF16, device=self.device)
            self._xg = buf
        return buf[:n]

    def identity_rows(self, n: int) -> torch.Tensor:
        """int32 [n] = 0..n-1: the row map of activations already in grouped order."""
        buf = getattr(self, "_ident", None)
        if buf is None or buf.numel() < n:
            buf = torch.arange(max(n, self.max_tokens * self.k), dtype=torch.int32, device=self.device)
            self._ident = buf
        return buf[:n]

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


# column width of the gate|up tile for each row-tile height of the grouped kernel
_GATEUP_COLS = {32: 128, 64: 128, 128: 128, 256: 128, 384: 64}


def shared_block_m(T: int, I: int) -> int:
    """Row-tile height of the shared experts' launch.  It runs on a side
    stream beside the routing and the routed experts, so it should read its
    weights as few times as possible and hold few CUs while the small routing
    and pack launches run: the tallest tile the shape allows (DeepSeek-V2-Lite
    mixed batch of 1304 tokens: 353 us per layer on 256-row tiles against
    376 us on 64-row tiles sized to fill the device alone, bit-identical)."""
    if I % _GATEUP_COLS[256] != 0:
        return 384
    return 32 if T <= 16 else 256


def shared_forward(x, shared_slot, ws: MoEWorkspace):
    """Always-on shared experts (DeepSeek-V2 `shared_experts`, one MLP of
    intermediate ws.shared_I applied to every token, unweighted): the grouped
    SwiGLU kernel with a single 'expert' whose rows are all T tokens in order.
    shared_slot: int64 [1] device table holding the shared gate|up|down block.
    Returns y_shared [T, H] bf16."""
    T = x.shape[0]
    H, Is = ws.H, ws.shared_I
    bm = shared_block_m(T, Is)
    if ws._shared_key != (T, bm):   # the one-expert tables depend only on T and the row tile
        ws.shared_offsets[1:].fill_(T)
        ws.shared_tiles[1:].fill_((T + bm - 1) // bm)
        ws._shared_key = (T, bm)
    ops.swiglu_grouped(x, ws.shared_rows[:T], ws.shared_offsets, ws.shared_sel, ws.shared_tiles,
                       (T + bm - 1) // bm, bm, shared_slot, H, Is, ws.h_shared, ws.y_shared)
    return ws.y_shared[:T]


def experts_resident(x, ids, weights, slots, ws: MoEWorkspace, out=None, *, block_m=None, add_in=None,
                     merge="fused", before_merge=None):
    """K4 (T == 1) or K2+K3+K5 (T > 1) over experts that are all addressable in `slots`.
    add_in [T, H] bf16 (shared-expert output) is added unweighted in the merge;
    before_merge() runs right before the merge is enqueued (to order add_in's producer).
    merge: 'fused' (fp32 sum, one rounding) or 'reference' (bf16 adds in
    ascending expert id, the reference runtime's default merge)."""
    T = x.shape[0]
    H, I, E, k = ws.H, ws.I, ws.E, ws.k
    out = ws.out[:T] if out is None else out
    if T == 1 and add_in is None:
        ops.swiglu_decode(x, ids, weights, slots, H, I, ws.h_ws, out, merge=merge)
        return out
    _, _, _, packed = ws.views(T)
    bm = block_m or ops.grouped_block_m((T * k) // E)
    bmd = down_block_m(bm, H, I)
    # the balanced schedule of all experts comes out of the pack launch
    sched = (ws.sel_all, bm, ws.sel_order, ws.tile_start) + ((bmd, ws.tile_start_down) if bmd != bm else ())
    ops.pack(ids, E, out=packed, workspace=ws.pack_ws, schedule=sched)
    grouped_ffn(x, packed, ws.sel_all, bm, (T * k + bm - 1) // bm + E, slots, ws,
                max_tiles_down=(T * k + bmd - 1) // bmd + E, scheduled=True)
    if before_merge is not None:
        before_merge()
    ops.merge(ws.y, packed.row_of, weights, out, add_in=add_in, mode=merge)
    return out


def down_block_m(bm: int, H: int, I: int) -> int:
    """Row tile of the down launch for a gate/up row tile `bm`: the 384-row
    gate/up tile is 128 columns wide, and the down projection (K = I) runs
    faster on 256x256 tiles that read each h row half as often (T=4096
    Qwen shape: 196 us against 222 us), where the shape allows them
    (H % 256 == 0, I % 128 == 0); other tiles are shared."""
    return 256 if bm == 384 and H % 256 == 0 and I % 128 == 0 else bm


def grouped_ffn(x, packed, sel, bm, max_tiles, slots, ws: MoEWorkspace, *, max_tiles_down, perm=None,
                scheduled=False):
    """Grouped SwiGLU over the experts in `sel` (int32 device): gate/up on
    bm-row tiles into ws.h_ws, down on down_block_m(bm, H, I)-row tiles into ws.y.
    max_tiles / max_tiles_down bound the two launches' tile counts.  perm
    (default packed.perm_token) maps grouped rows to rows of x.  scheduled:
    ws.sel_order / ws.tile_start (/ ws.tile_start_down) already hold the
    balanced schedule of `sel` (written by the pack launch)."""
    H, I = ws.H, ws.I
    perm = packed.perm_token if perm is None else perm
    nsel = sel.numel()
    tile_start, order = ws.tile_start[:nsel + 1], ws.sel_order[:nsel]
    bmd = down_block_m(bm, H, I)
    if bmd == bm:
        if not scheduled:
            ops.schedule(packed.counts, sel, bm, out=tile_start, order=order)
        ops.swiglu_grouped(x, perm, packed.offsets, order, tile_start, max_tiles, bm, slots, H, I, ws.h_ws, ws.y)
        return
    # one launch schedules both: the balanced order depends on the rows only
    tile_down = ws.tile_start_down[:nsel + 1]
    if not scheduled:
        ops.schedule(packed.counts, sel, bm, out=tile_start, order=order, block_m2=bmd, out2=tile_down)
    ops.swiglu_grouped_gateup(x, perm, packed.offsets, order, tile_start, max_tiles, bm, slots, H, I, ws.h_ws)
    ops.swiglu_grouped_down(ws.h_ws, packed.offsets, order, tile_down, max_tiles_down, bmd, slots, H, I, ws.y)


def moe_forward(x, gate, slots, ws: MoEWorkspace, *, normalize=True, bias=None, block_m=None, fused_decode=True,
                shared_slot=None, merge="fused", next_gate=None, pred_out=None):
    """Full layer: returns (out [T,H] bf16, logits, ids int32 [T,k], weights bf16 [T,k]).

    merge: 'fused' (each token's k weighted rows summed in fp32, one
    rounding) or 'reference' (added in ascending expert id in bf16
    arithmetic, bit-exact with the reference runtime's default merge).

    T == 1 runs the single-launch decode kernel (K4f) when the shape and the
    device allow it (fused_decode), else route (K1) + decode GEMV (K4).
    shared_slot (int64 [1] device table) adds always-on shared experts
    (DeepSeek-V2); the workspace must have been built with shared_I.
    next_gate / pred_out (T == 1 on the single-launch kernel only, see
    ops.decode_chained_supported): the next layer's gate-fallback prediction,
    top-k of next_gate . x, is written to pred_out [k] int32 by the same launch.
    """
    T = x.shape[0]
    if shared_slot is not None:
        if not ws.shared_I:
            raise ValueError("shared experts need a workspace built with shared_I")
        # the shared experts need only x: they run on a side stream beside the
        # routing and the routed experts (a one-expert launch alone does not
        # fill the device) and join before the merge adds their output
        cur = torch.cuda.current_stream(x.device)
        side = ws.side_stream()
        side.wait_stream(cur)
        with torch.cuda.stream(side):
            y_shared = shared_forward(x, shared_slot, ws)
        logits, ids, weights = route(x, gate, ws, normalize=normalize, bias=bias)
        out = experts_resident(x, ids, weights, slots, ws, block_m=block_m, add_in=y_shared, merge=merge,
                               before_merge=lambda: cur.wait_stream(side))
        return out, logits, ids, weights
    fused = (T == 1 and fused_decode and ws.k <= 8 and shared_slot is None
             and ops.decode_layer_supported(ws.H, ws.I, ws.E, ws.k, x.device))
    if (next_gate is None) != (pred_out is None):
        raise ValueError("next_gate and pred_out go together")
    if next_gate is not None and not (fused and ops.decode_chained_supported(ws.H, ws.I, ws.E, ws.k, x.device)):
        raise ValueError("the fused next-layer prediction needs one token on the single-launch decode kernel "
                         "with E <= H/2")
    if fused:
        logits, ids, weights, _ = ws.views(1)
        out = ws.out[:1]
        ops.decode_layer(x, gate, slots, ws.I, ws.k, normalize, bias=bias, out=out, logits=logits, ids=ids,
                         weights=weights, h_ws=ws.h_ws, merge=merge, next_gate=next_gate, pred_out=pred_out)
        return out, logits, ids, weights
    logits, ids, weights = route(x, gate, ws, normalize=normalize, bias=bias)
    out = experts_resident(x, ids, weights, slots, ws, block_m=block_m, merge=merge)
    return out, logits, ids, weights
