"""torch-tensor front end of the gfx950 MoE-layer kernels.

Each function checks shapes/dtypes/devices on the host, then calls the C-ABI
(include/pdscope_moe.h) on the current HIP stream of the tensors' device.
Tensors are borrowed; nothing here allocates unless an output is omitted.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib

BF16 = torch.bfloat16


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _need(t, name, dtype=None, ndim=None, device=None):
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must live on the GPU")
    if device is not None and t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if ndim is not None and t.ndim != ndim:
        raise ValueError(f"{name} must be {ndim}-D")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


_route_ws = {}


def route_workspace_size(T: int, H: int, E: int) -> int:
    return int(_lib.load().pdscope_route_workspace_size(int(T), int(H), int(E)))


def new_route_workspace(T: int, H: int, E: int, device) -> torch.Tensor:
    """Router scratch for up to T tokens: a zeroed counter (kept zero by the
    small-T kernel) followed by the split-K partial logits."""
    return torch.zeros(route_workspace_size(T, H, E), dtype=torch.uint8, device=device)


def route_workspace(device, T: int = 1, H: int = 16, E: int = 32) -> torch.Tensor:
    """Shared per-device router scratch, grown to cover (T, H, E) (not for
    graph capture: capture with a workspace you own)."""
    device = torch.device(device)
    if device.index is None:
        device = torch.device(device.type, torch.cuda.current_device())
    need = route_workspace_size(T, H, E)
    ws = _route_ws.get(device)
    if ws is None or ws.numel() < need:
        ws = torch.zeros(need, dtype=torch.uint8, device=device)
        _route_ws[device] = ws
    return ws


def slot_table(tensors, device) -> torch.Tensor:
    """Device int64 table of expert base addresses (gate|up|down blocks)."""
    return torch.tensor([t.data_ptr() for t in tensors], dtype=torch.int64, device=device)


# --------------------------------------------------------------------- A1/A2

def route_topk(x, gate, top_k, normalize, *, bias=None, capture_probabilities=False, out=None, workspace=None):
    """K1 router.  Returns (logits bf16 [T,E], ids int32 [T,k], weights bf16 [T,k], probs|None)."""
    _need(x, "inputs", BF16, 2)
    _need(gate, "gate", BF16, 2, x.device)
    T, H = x.shape
    E = gate.shape[0]
    if gate.shape[1] != H:
        raise ValueError("router input shape/dtype mismatch")
    if type(top_k) is not int or not 0 < top_k <= E:
        raise ValueError("invalid routing parameters")
    if bias is not None:
        _need(bias, "bias", torch.float32, 1, x.device)
        if bias.numel() != E:
            raise ValueError("bias must have one entry per expert")
    if out is None:
        logits = torch.empty((T, E), dtype=BF16, device=x.device)
        ids = torch.empty((T, top_k), dtype=torch.int32, device=x.device)
        weights = torch.empty((T, top_k), dtype=BF16, device=x.device)
    else:
        logits, ids, weights = out
    probs = torch.empty((T, E), dtype=torch.float32, device=x.device) if capture_probabilities else None
    if workspace is None:
        workspace = route_workspace(x.device, T, H, E)
    elif workspace.numel() < route_workspace_size(T, H, E):
        raise ValueError("router workspace too small for this token count")
    _lib.call("pdscope_route_topk", _p(x), _p(gate), _p(bias), T, H, E, top_k, int(bool(normalize)),
              _p(logits), _p(ids), _p(weights), _p(probs), _p(workspace), _stream(x.device))
    return logits, ids, weights, probs


def route_hist(ids, E, out=None):
    _need(ids, "ids", torch.int32)
    hist = out if out is not None else torch.empty(E, dtype=torch.int32, device=ids.device)
    _lib.call("pdscope_route_hist", _p(ids), ids.numel(), E, _p(hist), _stream(ids.device))
    return hist


# --------------------------------------------------------------------- A3

@dataclass
class Packed:
    counts: torch.Tensor      # int32 [E]
    offsets: torch.Tensor     # int32 [E+1]
    perm_token: torch.Tensor  # int32 [T*k]
    perm_pos: torch.Tensor    # int32 [T*k]
    row_of: torch.Tensor      # int32 [T*k]


def pack_workspace_size(T: int, k: int, E: int) -> int:
    return int(_lib.load().pdscope_pack_workspace_size(int(T), int(k), int(E)))


def pack(ids, E, out: Packed | None = None, workspace=None, *, schedule=None) -> Packed:
    """K2 grouping.  schedule=(sel, block_m, order, tile_start[, block_m2,
    tile_start2]) also writes the balanced schedule of `sel` over the
    resulting counts (as schedule(..., order=...)) from inside the pack
    launch (pdscope_pack_schedule_balanced)."""
    _need(ids, "ids", torch.int32, 2)
    T, k = ids.shape
    dev = ids.device
    n = T * k
    if out is None:
        out = Packed(torch.empty(E, dtype=torch.int32, device=dev), torch.empty(E + 1, dtype=torch.int32, device=dev),
                     torch.empty(n, dtype=torch.int32, device=dev), torch.empty(n, dtype=torch.int32, device=dev),
                     torch.empty(n, dtype=torch.int32, device=dev))
    need = pack_workspace_size(T, k, E)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    args = (_p(ids), T, k, E, _p(out.counts), _p(out.offsets), _p(out.perm_token), _p(out.perm_pos), _p(out.row_of),
            _p(workspace) if need else None)
    if schedule is None:
        _lib.call("pdscope_pack", *args, _stream(dev))
        return out
    sel, block_m, order, tile_start, *second = schedule
    block_m2, tile_start2 = second if second else (0, None)
    for t, name, size in ((sel, "sel", 0), (order, "order", sel.numel()), (tile_start, "tile_start", sel.numel() + 1)):
        _need(t, name, torch.int32, 1, dev)
        if t.numel() < size:
            raise ValueError(f"{name} smaller than sel needs")
    if tile_start2 is not None:
        _need(tile_start2, "tile_start2", torch.int32, 1, dev)
        if tile_start2.numel() < sel.numel() + 1:
            raise ValueError("tile_start2 smaller than sel needs")
    _lib.call("pdscope_pack_schedule_balanced", *args, _p(sel), sel.numel(), block_m, block_m2, _p(order),
              _p(tile_start), _p(tile_start2), _stream(dev))
    return out


_static_ready = set()


def pack_static_max_ids(device=None) -> int:
    """The id limit of pack_static; also looks up the library's static
    scratch on `device` (default: the current one), so a caller that sizes
    its inputs at set-up pays that lookup outside any graph capture."""
    device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    if device.index is None:
        device = torch.device(device.type, torch.cuda.current_device())
    with torch.cuda.device(device):
        n = int(_lib.load().pdscope_pack_static_max_ids())
    if n == 0:
        raise _lib.PDScopeError("pdscope_pack_static_max_ids: " + _lib.load().pdscope_last_error().decode())
    _static_ready.add(device)
    return n


def pack_static(ids, E, out: Packed) -> Packed:
    """pack() through the entry point that allocates nothing (its multi-block
    scratch is a library-owned device array; calls overlapping in time on
    one GPU race).  All outputs are caller-provided.  The first call on a
    device looks the scratch up (pack_static_max_ids) unless that was done."""
    _need(ids, "ids", torch.int32, 2)
    T, k = ids.shape
    dev = ids.device
    if dev not in _static_ready:
        pack_static_max_ids(dev)
    for t, n, size in ((out.counts, "counts", E), (out.offsets, "offsets", E + 1), (out.perm_token, "perm_token", T * k),
                       (out.perm_pos, "perm_pos", T * k), (out.row_of, "row_of", T * k)):
        _need(t, n, torch.int32, None, dev)
        if t.numel() < size:
            raise ValueError(f"{n} holds {t.numel()} entries, needs {size}")
    _lib.call("pdscope_pack_static", _p(ids), T, k, E, _p(out.counts), _p(out.offsets), _p(out.perm_token),
              _p(out.perm_pos), _p(out.row_of), _stream(dev))
    return out


def grouped_block_m(rows_hint: int, max_rows: int | None = None) -> int:
    """Row tile of the grouped SwiGLU launch for rows_hint mean rows per expert
    (and, when the host knows it, the largest expert's rows)."""
    if max_rows is None:
        return int(_lib.load().pdscope_grouped_block_m(int(rows_hint)))
    return int(_lib.load().pdscope_grouped_block_m_max(int(rows_hint), int(max_rows)))


def schedule(counts, sel, block_m, out=None, order=None, *, block_m2=None, out2=None):
    """Tile prefix over `sel` (order=None), or, with an int32 [nsel] `order`
    buffer, the balanced order of pdscope_schedule_balanced and the prefix
    over it: the grouped launch must then take `order` as its sel.  A sel
    entry outside [0, counts.numel()) counts as an expert with no rows.  With
    block_m2 and out2 (balanced only), out2 receives the same order's prefix
    for a second row tile, from the same launch."""
    _need(counts, "counts", torch.int32, 1)
    _need(sel, "sel", torch.int32, 1, counts.device)
    tile_start = out if out is not None else torch.empty(sel.numel() + 1, dtype=torch.int32, device=counts.device)
    if block_m2 is not None:
        if order is None or out2 is None:
            raise ValueError("a second row tile needs the balanced order and an out2 buffer")
        _need(order, "order", torch.int32, 1, counts.device)
        _need(out2, "out2", torch.int32, 1, counts.device)
        if order.numel() < sel.numel() or out2.numel() < sel.numel() + 1:
            raise ValueError("order / out2 buffers smaller than sel")
        _lib.call("pdscope_schedule_balanced_pair", _p(counts), counts.numel(), _p(sel), sel.numel(), block_m,
                  block_m2, _p(order), _p(tile_start), _p(out2), _stream(counts.device))
        return tile_start
    if order is None:
        _lib.call("pdscope_schedule", _p(counts), counts.numel(), _p(sel), sel.numel(), block_m, _p(tile_start),
                  _stream(counts.device))
    else:
        _need(order, "order", torch.int32, 1, counts.device)
        if order.numel() < sel.numel():
            raise ValueError("order buffer smaller than sel")
        _lib.call("pdscope_schedule_balanced", _p(counts), counts.numel(), _p(sel), sel.numel(), block_m, _p(order),
                  _p(tile_start), _stream(counts.device))
    return tile_start


# --------------------------------------------------------------------- A4

def swiglu_grouped(x, perm_token, offsets, sel, tile_start, max_tiles, block_m, slots, H, I, h_ws, y):
    _need(x, "inputs", BF16, 2)
    dev = x.device
    for t, n in ((perm_token, "perm_token"), (offsets, "offsets"), (sel, "sel"), (tile_start, "tile_start")):
        _need(t, n, torch.int32, 1, dev)
    _need(slots, "slots", torch.int64, 1, dev)
    _need(h_ws, "h_ws", BF16, None, dev)
    _need(y, "y", BF16, None, dev)
    if h_ws.numel() < perm_token.numel() * I or y.numel() < perm_token.numel() * H:
        raise ValueError("h_ws / y workspaces are smaller than rows x I / rows x H")
    _lib.call("pdscope_swiglu_grouped", _p(x), _p(perm_token), _p(offsets), _p(sel), sel.numel(), _p(tile_start),
              int(max_tiles), int(block_m), _p(slots), H, I, _p(h_ws), _p(y), _stream(dev))
    return y


def swiglu_grouped_gateup(x, perm_token, offsets, sel, tile_start, max_tiles, block_m, slots, H, I, h_ws):
    """Only the gate/up + SwiGLU launch of swiglu_grouped (K3, first half)."""
    dev = x.device
    _need(x, "inputs", BF16, 2)
    _need(h_ws, "h_ws", BF16, None, dev)
    if h_ws.numel() < perm_token.numel() * I:
        raise ValueError("h_ws is smaller than rows x I")
    _lib.call("pdscope_swiglu_grouped_gateup", _p(x), _p(perm_token), _p(offsets), _p(sel), sel.numel(),
              _p(tile_start), int(max_tiles), int(block_m), _p(slots), H, I, _p(h_ws), _stream(dev))


def swiglu_grouped_down(h_ws, offsets, sel, tile_start, max_tiles, block_m, slots, H, I, y):
    """Only the down-projection launch of swiglu_grouped (K3, second half)."""
    dev = h_ws.device
    _need(y, "y", BF16, None, dev)
    _lib.call("pdscope_swiglu_grouped_down", _p(h_ws), _p(offsets), _p(sel), sel.numel(), _p(tile_start),
              int(max_tiles), int(block_m), _p(slots), H, I, _p(y), _stream(dev))


MERGE_MODES = {"fused": 0, "reference": 1}


def merge_mode(merge: str) -> int:
    """C-ABI merge_mode of a runtime merge name: 'fused' (fp32, one rounding)
    or 'reference' (bf16 adds in ascending expert id, the reference's default)."""
    if merge not in MERGE_MODES:
        raise ValueError("invalid merge mode")
    return MERGE_MODES[merge]


def swiglu_decode(x, ids, w, slots, H, I, h_ws, out, *, merge="fused"):
    _need(x, "inputs", BF16)
    dev = x.device
    _need(ids, "ids", torch.int32, None, dev)
    _need(w, "weights", BF16, None, dev)
    _need(slots, "slots", torch.int64, 1, dev)
    _need(h_ws, "h_ws", BF16, None, dev)
    _need(out, "out", BF16, None, dev)
    k = ids.numel()
    if x.numel() != H or out.numel() != H or w.numel() != k or h_ws.numel() < k * I:
        raise ValueError("decode expects one token: x/out [H], ids/weights [k], h_ws >= k*I")
    _lib.call("pdscope_swiglu_decode", _p(x), _p(ids), _p(w), k, _p(slots), H, I, _p(h_ws), _p(out),
              merge_mode(merge), _stream(dev))
    return out


_decode_ws = {}
_decode_ok = {}


DECODE_WS_ERROR_WORD = 1024


def decode_workspace(device, H) -> torch.Tensor:
    """Zero-filled hand-off words of the fused decode kernel for hidden size H
    on `device` (its per-block epochs assume one grid size, i.e. one H, and
    launches on one stream at a time)."""
    device = torch.device(device)
    if device.index is None:
        device = torch.device(device.type, torch.cuda.current_device())
    key = (device, int(H))
    ws = _decode_ws.get(key)
    if ws is None:
        n = int(_lib.load().pdscope_decode_workspace_bytes())
        ws = torch.zeros(n // 4, dtype=torch.int32, device=key[0])
        _decode_ws[key] = ws
    return ws


def decode_workspace_error(device, H) -> int:
    """Sticky error word of the fused decode kernel (non-zero after a bounded wait gave up)."""
    return int(decode_workspace(device, H)[DECODE_WS_ERROR_WORD].item())


def decode_layer_supported(H, I, E, k, device) -> bool:
    device = torch.device(device)
    if device.index is None:
        device = torch.device(device.type, torch.cuda.current_device())
    key = (device, H, I, E, k)
    ok = _decode_ok.get(key)
    if ok is None:
        with torch.cuda.device(key[0]):
            ok = bool(_lib.load().pdscope_decode_layer_supported(H, I, E, k))
        _decode_ok[key] = ok
    return ok


_chain_ok = {}


def decode_chained_supported(H, I, E, k, device, *, predictor=True) -> bool:
    """Whether the chained single-launch decode kernel (residual input and/or
    next-layer prediction) runs this shape on `device`: its grid must be
    co-resident, which the chained variant's extra registers and LDS can
    prevent where the plain kernel fits."""
    device = torch.device(device)
    if device.index is None:
        device = torch.device(device.type, torch.cuda.current_device())
    key = (device, H, I, E, k, bool(predictor))
    ok = _chain_ok.get(key)
    if ok is None:
        with torch.cuda.device(key[0]):
            ok = bool(_lib.load().pdscope_decode_layer_chained_supported(H, I, E, k, int(bool(predictor))))
        _chain_ok[key] = ok
    return ok


def decode_layer(x, gate, slots, I, top_k, normalize, *, bias=None, out, logits, ids, weights, h_ws, probs=None,
                 merge="fused", resid=None, x_out=None, next_gate=None, pred_out=None):
    """K4f: route + top-k + SwiGLU GEMV + down/merge of one token in one launch.

    Chain arguments (pdscope_decode_layer_chained): the input is
    bf16(x + resid) when `resid` is given (written to `x_out`); with
    `next_gate`, `pred_out` receives the next layer's gate-fallback
    prediction top-k(next_gate . input)."""
    _need(x, "inputs", BF16)
    dev = x.device
    _need(gate, "gate", BF16, 2, dev)
    _need(slots, "slots", torch.int64, 1, dev)
    E, H = gate.shape
    if x.numel() != H or out.numel() != H or logits.numel() != E or ids.numel() != top_k or weights.numel() != top_k:
        raise ValueError("decode_layer expects one token: x/out [H], logits [E], ids/weights [k]")
    if h_ws.numel() < top_k * I or slots.numel() < E:
        raise ValueError("decode_layer: h_ws must hold k*I values and slots E entries")
    _need(ids, "ids", torch.int32, None, dev)
    for t, n in ((out, "out"), (logits, "logits"), (weights, "weights"), (h_ws, "h_ws")):
        _need(t, n, BF16, None, dev)
    if bias is not None:
        _need(bias, "bias", torch.float32, 1, dev)
    if probs is not None:
        _need(probs, "probs", torch.float32, None, dev)
    chained = any(t is not None for t in (resid, x_out, next_gate, pred_out))
    if not chained:
        _lib.call("pdscope_decode_layer", _p(x), _p(gate), _p(bias), H, E, top_k, int(bool(normalize)),
                  merge_mode(merge), _p(slots), I,
                  _p(logits), _p(ids), _p(weights), _p(probs), _p(h_ws), _p(out), _p(decode_workspace(dev, H)),
                  _stream(dev))
        return out
    if (resid is None) != (x_out is None):
        raise ValueError("decode_layer: resid and x_out go together")
    if (next_gate is None) != (pred_out is None):
        raise ValueError("decode_layer: next_gate and pred_out go together")
    for t, n in ((resid, "resid"), (x_out, "x_out")):
        if t is not None:
            _need(t, n, BF16, None, dev)
            if t.numel() != H:
                raise ValueError(f"decode_layer: {n} must hold H values")
    if pred_out is not None:
        _need(pred_out, "pred_out", torch.int32, None, dev)
        if pred_out.numel() != top_k:
            raise ValueError("decode_layer: pred_out must hold k ids")
    if next_gate is not None:
        _need(next_gate, "next_gate", BF16, 2, dev)
        if tuple(next_gate.shape) != (E, H):
            raise ValueError("decode_layer: next_gate must be [E, H] like gate")
    _lib.call("pdscope_decode_layer_chained", _p(x), _p(resid), _p(x_out), _p(gate), _p(bias), H, E, top_k,
              int(bool(normalize)), merge_mode(merge), _p(slots), I, _p(next_gate), _p(pred_out),
              _p(logits), _p(ids), _p(weights), _p(probs), _p(h_ws), _p(out), _p(decode_workspace(dev, H)),
              _stream(dev))
    return out


class DecodeBinding:
    """One resident decode layer bound once (pdscope_decode_bind): its gate,
    slot table (by address: refresh the contents, not the tensor), optional
    next-layer gate and logit bias are checked and planned at construction,
    and each token is then one C call, numbered seq (1 .. 32767), that
    launches the fused decode kernel and a one-wave read-back kernel (host:
    pinned int32 CPU tensor).  The decode kernel stores (seq << 16) | id of
    the routed ids into host[ids_at:ids_at+k] as soon as its routing is final
    (before it completes), and of the next-layer prediction into
    host[ids_at+k:ids_at+2k]; the read-back kernel then stores (seq << 16) |
    the kernel's sticky error word into host[error_at].  A word is valid
    once it carries seq in its upper half; a tagged host[error_at] also
    means that the decode launch has completed.  tagged_words() decodes.

    The binding owns its device scratch (int32 ids, prediction, h) and keeps
    every tensor it bound alive.  Calls on one device share the fused
    kernel's workspace, so they must be ordered on one stream."""

    def __init__(self, gate, slots, I, top_k, normalize, *, host, error_at, ids_at=0, merge="fused",
                 next_gate=None, bias=None):
        dev = gate.device
        _need(gate, "gate", BF16, 2, dev)
        _need(slots, "slots", torch.int64, 1, dev)
        E, H = gate.shape
        k = int(top_k)
        if slots.numel() < E or not slots.is_contiguous():
            raise ValueError("DecodeBinding: slots must be a contiguous table of E entries")
        if next_gate is not None:
            _need(next_gate, "next_gate", BF16, 2, dev)
            if tuple(next_gate.shape) != (E, H) or not next_gate.is_contiguous():
                raise ValueError("DecodeBinding: next_gate must be a contiguous [E, H] tensor like gate")
        if not gate.is_contiguous():
            raise ValueError("DecodeBinding: gate must be contiguous")
        if bias is not None:
            _need(bias, "bias", torch.float32, 1, dev)
            if bias.numel() != E:
                raise ValueError("DecodeBinding: bias must hold E values")
        if (not isinstance(host, torch.Tensor) or host.device.type != "cpu" or host.dtype != torch.int32
                or not host.is_pinned() or not host.is_contiguous()):
            raise ValueError("DecodeBinding: host must be a contiguous pinned int32 CPU tensor")
        if not (0 <= ids_at and ids_at + 2 * k <= host.numel() and 0 <= error_at < host.numel()
                and not ids_at <= error_at < ids_at + 2 * k):
            raise ValueError("DecodeBinding: read-back words outside host or overlapping")
        self.H, self.E, self.I, self.k = H, E, int(I), k
        self.device = dev
        self.ids = torch.zeros(k, dtype=torch.int32, device=dev)
        self.pred = torch.full((k,), -1, dtype=torch.int32, device=dev) if next_gate is not None else None
        self.h_ws = torch.empty(k * self.I, dtype=BF16, device=dev)
        self.workspace = decode_workspace(dev, H)
        self._refs = (gate, slots, next_gate, bias, host)
        lib = _lib.load()
        handle = ctypes.c_void_p()
        base = host.data_ptr()
        with torch.cuda.device(dev):
            rc = lib.pdscope_decode_bind(_p(gate), _p(bias), H, E, k, int(bool(normalize)), merge_mode(merge),
                                         _p(slots), self.I, _p(next_gate), _p(self.pred), _p(self.ids), None,
                                         _p(self.h_ws), _p(self.workspace), base + 4 * ids_at, base + 4 * error_at,
                                         ctypes.byref(handle))
        if rc != 0:
            _lib.raise_for("pdscope_decode_bind", rc)
        self._handle = handle.value
        self._run = lib.pdscope_decode_run
        self._unbind = lib.pdscope_decode_unbind

    @staticmethod
    def tagged_words(words, seq):
        """The values of read-back words (a sequence of int32) if every one
        carries seq in its upper half, else None."""
        vals = []
        for w in words:
            w = int(w)
            if w >> 16 != seq:
                return None
            vals.append(w & 0xFFFF)
        return vals

    def run_ptrs(self, x, out, logits, weights, selected, seq, stream):
        """The per-token call on raw addresses (x [H], out [H], logits [E],
        weights [k] bf16, selected [k] int64 or 0), its sequence number
        (1 .. 32767, the tag of its read-back words) and a raw hipStream_t,
        for callers that checked the tensors themselves."""
        rc = self._run(self._handle, x, out, logits, weights, selected, seq, stream)
        if rc != 0:
            _lib.raise_for("pdscope_decode_run", rc)

    def run(self, x, out, logits, weights, selected=None, stream=None, seq=1):
        """One token: x [1,H] bf16 in; out [1,H], logits [1,E], weights [1,k]
        bf16 and optionally selected [1,k] int64 out, on `stream` (default:
        the current stream of the binding's device); the read-back words carry
        `seq` (1 .. 32767)."""
        if self._handle is None:
            raise ValueError("DecodeBinding is closed")
        dev = self.device
        for t, n, dt, size in ((x, "x", BF16, self.H), (out, "out", BF16, self.H), (logits, "logits", BF16, self.E),
                               (weights, "weights", BF16, self.k)):
            _need(t, n, dt, None, dev)
            if t.numel() != size or not t.is_contiguous():
                raise ValueError(f"DecodeBinding.run: {n} must be a contiguous tensor of {size} values")
        if selected is not None:
            _need(selected, "selected", torch.int64, None, dev)
            if selected.numel() != self.k or not selected.is_contiguous():
                raise ValueError("DecodeBinding.run: selected must be a contiguous tensor of k values")
        s = torch.cuda.current_stream(dev) if stream is None else stream
        self.run_ptrs(x.data_ptr(), out.data_ptr(), logits.data_ptr(), weights.data_ptr(),
                      0 if selected is None else selected.data_ptr(), int(seq), s.cuda_stream)

    def close(self):
        if self._handle is not None:
            self._unbind(self._handle)
            self._handle = None
            self._refs = ()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# --------------------------------------------------------------------- A8/A9

def merge(y, row_of, w, out, add_in=None, *, mode="fused"):
    _need(w, "weights", BF16, 2)
    dev = w.device
    _need(y, "y", BF16, None, dev)
    _need(row_of, "row_of", torch.int32, 1, dev)
    _need(out, "out", BF16, 2, dev)
    T, k = w.shape
    H = out.shape[1]
    if add_in is not None:
        _need(add_in, "add_in", BF16, 2, dev)
    name = "pdscope_merge_ordered" if merge_mode(mode) else "pdscope_merge"
    _lib.call(name, _p(y), _p(row_of), _p(w), T, k, H, _p(add_in), _p(out), _stream(dev))
    return out


def stage_expert(dst, src, *, event=None, stream=None):
    """One H2D copy of a pinned expert block into a device slot, then `event` on the same stream.

    The torch event is recorded by torch after the copy is enqueued (its HIP
    event only exists once recorded), so completion of that event implies the
    copy landed.
    """
    if src.device.type != "cpu" or not src.is_pinned():
        raise ValueError("staging source must be page-locked host memory")
    nbytes = src.numel() * src.element_size()
    if dst.numel() * dst.element_size() < nbytes:
        raise ValueError("staging slot is smaller than the expert block")
    s = stream if stream is not None else torch.cuda.current_stream(dst.device)
    _lib.call("pdscope_stage_expert", _p(dst), _p(src), nbytes, None, ctypes.c_void_p(s.cuda_stream))
    if event is not None:
        event.record(s)


def stage_merge(host_block_ptr, rows, row_bytes, scratch, out, tokens, weights):
    _need(scratch, "scratch", BF16, None)
    dev = scratch.device
    _need(out, "out", BF16, None, dev)
    _need(tokens, "tokens", torch.int64, 1, dev)
    _need(weights, "weights", BF16, None, dev)
    if scratch.numel() * 2 != rows * row_bytes:
        raise RuntimeError("scratch buffer must match the packed block")
    if out.dim() != 2 or out.shape[1] * 2 != row_bytes or tokens.numel() != rows or weights.numel() != rows:
        raise RuntimeError("out must be [tokens, row_bytes / 2]; tokens and weights one entry per row")
    _lib.call("pdscope_stage_merge", ctypes.c_void_p(int(host_block_ptr)), int(rows), int(row_bytes), _p(scratch),
              _p(out), _p(tokens), _p(weights), int(out.shape[0]), _stream(dev))
    return out
