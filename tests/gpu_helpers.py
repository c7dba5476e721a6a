"""Shared helpers for the GPU parity tests."""
import numpy as np
import torch


def u16(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> numpy uint16 bit patterns (on the host)."""
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16).copy()


def from_u16(a: np.ndarray, device="cuda") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(device)


def ulp_diff_bf16(a, b):
    a = a.astype(np.int32)
    b = b.astype(np.int32)
    fa = np.where(a & 0x8000, -(a & 0x7FFF), a & 0x7FFF)
    fb = np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)
    return np.abs(fa - fb)


def err_metrics(actual_f32: np.ndarray, ref_f32: np.ndarray):
    """max rel err := max|d| / max|ref|; mean abs err; rel-L2 (benchmarks/harness.py:33-43)."""
    d = actual_f32.astype(np.float64) - ref_f32.astype(np.float64)
    ref = ref_f32.astype(np.float64)
    return dict(max_rel=float(np.abs(d).max() / max(np.abs(ref).max(), 1e-30)),
                mean_abs=float(np.abs(d).mean()),
                rel_l2=float(np.linalg.norm(d) / max(np.linalg.norm(ref), 1e-30)))


# tolerance of the layer path vs the reference expert path (bf16, fp32 accumulate)
MAX_REL = 1e-2
MEAN_ABS = 1e-3


def logits_within_accumulation_error(kern, orc_exact, x_u16, gate_u16, bf16_to_f32):
    """Kernel logits (fp32 accumulate, any order) vs exactly rounded logits:
    every mismatch is one bf16 ulp, or within n*2^-24*sum|x*w| near zero."""
    d = ulp_diff_bf16(kern, orc_exact)
    if (d == 0).all():
        return True, 0
    xf = bf16_to_f32(x_u16).astype(np.float64)
    gf = bf16_to_f32(gate_u16).astype(np.float64)
    bound = xf.shape[1] * 2.0 ** -24 * (np.abs(xf) @ np.abs(gf).T)
    diff = np.abs(bf16_to_f32(kern).astype(np.float64) - bf16_to_f32(orc_exact))
    ok = bool(np.all((d <= 1) | (diff <= bound)))
    return ok, int((d > 0).sum())


def oracle_layer_given_routing(orc, x_u16, ids, w_u16, experts_u16, H, I, merge="fused"):
    """Oracle expert path + merge for a given routing (ids int [T,k], weights bf16 bits).
    merge "fused" is the exactly rounded weighted sum, "reference" the
    reference's bf16 index_add_ in ascending expert id."""
    E = experts_u16.shape[0]
    p = orc.pack(np.ascontiguousarray(ids, dtype=np.int32), E)
    xg = x_u16[p["perm_token"]]
    y = np.empty((ids.size, H), np.uint16)
    IH = I * H
    for e in np.nonzero(p["counts"])[0]:
        a, b = p["offsets"][e], p["offsets"][e + 1]
        blk = experts_u16[e]
        y[a:b] = orc.expert_forward(xg[a:b], blk[:IH].reshape(I, H), blk[IH:2 * IH].reshape(I, H),
                                    blk[2 * IH:].reshape(H, I))
    if merge not in ("fused", "reference"):
        raise ValueError(merge)
    mrg = orc.merge if merge == "fused" else orc.merge_ordered
    return mrg(y, p["row_of"], w_u16), y, p


def oracle_tokens_given_routing(orc, x_u16, ids, w_u16, tokens, block_of, H, I, add_in=None, merge="fused"):
    """Oracle layer output of selected tokens for a given routing.

    block_of(e) returns expert e's flat gate|up|down block as uint16.  The
    rows of one expert go through the oracle in one call.  merge "fused" is
    the exactly rounded weighted sum, "reference" the reference's bf16
    index_add_ in ascending expert id (the runtime's default merge).
    Returns (out [n,H], y [n*k,H]) with y in (token, slot) order."""
    tokens = np.asarray(tokens)
    n, k = len(tokens), ids.shape[1]
    y = np.empty((n * k, H), np.uint16)
    sel = ids[tokens]
    IH = I * H
    for e in np.unique(sel):
        where = np.argwhere(sel == e)
        xs = np.ascontiguousarray(x_u16[tokens[where[:, 0]]])
        blk = block_of(int(e))
        y[where[:, 0] * k + where[:, 1]] = orc.expert_forward(
            xs, blk[:IH].reshape(I, H), blk[IH:2 * IH].reshape(I, H), blk[2 * IH:].reshape(H, I))
    w_t = np.ascontiguousarray(w_u16[tokens])
    if merge == "fused":
        row_of = np.arange(n * k, dtype=np.int32).reshape(n, k)
        return orc.merge(y, row_of, w_t, add_in=add_in), y
    if merge != "reference":
        raise ValueError(merge)
    # merge_ordered adds a token's rows in grouped-row order, which is
    # ascending expert id: place each token's rows by the rank of their id
    rank = np.argsort(np.argsort(sel, axis=1, kind="stable"), axis=1, kind="stable")
    row_of = (np.arange(n)[:, None] * k + rank).astype(np.int32)
    y_rows = np.empty_like(y)
    y_rows[row_of.reshape(-1)] = y
    return orc.merge_ordered(y_rows, row_of, w_t, add_in=add_in), y


def assert_layer_close(orc, out, ref_u16):
    m = err_metrics(orc.bf16_to_f32(u16(out)), orc.bf16_to_f32(ref_u16))
    assert m["max_rel"] <= MAX_REL and m["mean_abs"] <= MEAN_ABS, m
    return m
