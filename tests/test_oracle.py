"""Pin the C oracle (CPU only).

Each oracle function is checked against something that does not restate its
own formula: the torch-CPU golden fixtures (tests/golden/make_golden.py),
brute force on tiny inputs, closed forms, and invariants.  Several tests plant
a plausible mistake (in the oracle's inputs/arguments, on the CPU) and assert
that the same check then fails, so the pins are known to bite.
"""
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    return dict(np.load(GOLDEN / f"{name}.npz", allow_pickle=False))


def ulp_diff_bf16(a, b):
    a = a.astype(np.int32)
    b = b.astype(np.int32)
    # sign-magnitude -> monotone integer line
    fa = np.where(a & 0x8000, -(a & 0x7FFF), a & 0x7FFF)
    fb = np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)
    return np.abs(fa - fb)


# ------------------------------------------------------------------ codecs

def test_f32_to_bf16_matches_torch(orc):
    import torch
    rng = np.random.default_rng(1)
    v = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 100000),
                        np.array([0.0, -0.0, 1.0, 65504.0, 3.0e38, -3.0e38, 1e-40], np.float32)]).astype(np.float32)
    ours = orc.f32_to_bf16(v)
    theirs = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    assert np.array_equal(orc.bf16_to_f32(ours), torch.from_numpy(v).to(torch.bfloat16).float().numpy())


def _bf16_correct_round(d: float) -> int:
    """Brute force: nearest bf16 (ties to even) by exact rational comparison."""
    import struct
    f = Fraction(d)
    u32 = struct.unpack("<I", struct.pack("<f", np.float32(d)))[0]
    c = (u32 >> 16) & 0xFFFF
    best = None
    for cand in range((c - 2) & 0xFFFF, (c + 3)):
        cand &= 0xFFFF
        if (cand & 0x7F80) == 0x7F80:
            continue
        val = Fraction(float(np.uint32(cand << 16).view(np.float32)))
        key = (abs(val - f), cand & 1)
        if best is None or key < best[0]:
            best = (key, cand)
    return best[1]


def test_f64_to_bf16_is_one_correct_rounding(orc):
    rng = np.random.default_rng(2)
    vals = list(rng.standard_normal(3000) * 10.0 ** rng.integers(-5, 5, 3000))
    # exact midpoints and near-midpoints between bf16 neighbours: where a naive
    # f64->f32->bf16 double rounding would go wrong
    for base in rng.integers(0x3C00, 0x4300, 200):
        lo = float(np.uint32(int(base) << 16).view(np.float32))
        hi = float(np.uint32((int(base) + 1) << 16).view(np.float32))
        mid = (lo + hi) / 2
        vals += [mid, np.nextafter(mid, np.inf), np.nextafter(mid, -np.inf), mid + (hi - lo) * 2 ** -30]
    for d in vals:
        assert orc.f64_to_bf16_scalar(d) == _bf16_correct_round(float(d)), d


def test_naive_double_rounding_would_fail(orc):
    """Planted mistake: rounding f64->f32 (nearest) then f32->bf16 is not a
    single rounding; the brute-force check above must catch it."""
    d = float(np.uint32(0x3F808000).view(np.float32)) + 2.0 ** -40  # just above a bf16 midpoint
    naive = int(orc.f32_to_bf16(np.array([d], np.float32))[0])
    assert naive != _bf16_correct_round(d)
    assert orc.f64_to_bf16_scalar(d) == _bf16_correct_round(d)


def test_expf_accuracy(orc):
    import math
    xs = np.concatenate([-np.linspace(0, 87, 20001), -np.random.default_rng(3).random(5000) * 20,
                         [0.0, -1e-8, -0.34657, -0.34658, -86.0]])
    worst = 0.0
    for x in xs.astype(np.float32):
        got = orc.expf(float(x))
        want = math.exp(float(x))
        if want < 2.0 ** -125 * 1.5:
            assert got == 0.0 or abs(got - want) / want < 1e-6
            continue
        worst = max(worst, abs(got - want) / want)
    assert orc.expf(0.0) == 1.0
    assert worst < 2.5e-7, worst        # within ~2 fp32 ulp
    assert orc.expf(-200.0) == 0.0 and orc.expf(float("-inf")) == 0.0


# ------------------------------------------------------------------ route

ROUTE_CASES = ["qwen_t64", "qwen_t1", "ties_t128", "dsv2_t48", "zipf_t64"]


@pytest.mark.parametrize("name", ROUTE_CASES)
def test_route_logits_vs_torch(orc, name):
    g = load(f"route_{name}")
    T, H, E, k, norm = g["meta"]
    ours = orc.route_logits(g["x"].reshape(T, H), g["gate"].reshape(E, H))
    d = ulp_diff_bf16(ours, g["logits"])
    # torch accumulates in fp32 (order unspecified), the oracle rounds the
    # exact sum.  A mismatch is one bf16 ulp, or (near zero, after
    # cancellation) within the fp32 accumulation error bound n*2^-24*sum|x*w|.
    xf = orc.bf16_to_f32(g["x"]).reshape(T, H).astype(np.float64)
    gf = orc.bf16_to_f32(g["gate"]).reshape(E, H).astype(np.float64)
    bound = H * 2.0 ** -24 * (np.abs(xf) @ np.abs(gf).T)
    diff = np.abs(orc.bf16_to_f32(ours).astype(np.float64) - orc.bf16_to_f32(g["logits"]))
    assert np.all((d <= 1) | (diff <= bound))
    assert (d > 0).mean() < 2e-3


@pytest.mark.parametrize("name", ROUTE_CASES)
def test_route_ids_bit_exact_given_logits(orc, name):
    g = load(f"route_{name}")
    T, H, E, k, norm = (int(v) for v in g["meta"])
    ids, w, probs = orc.route_from_logits(g["logits"], k, bool(norm), g.get("bias"), want_probs=True)
    assert np.array_equal(ids, g["ids"])
    du = ulp_diff_bf16(w, g["weights"])
    assert du.max() <= 1 and (du > 0).mean() < 0.02
    rel = np.abs(probs - g["probs"]) / np.maximum(g["probs"], 1e-30)
    assert rel.max() < 2e-6


def test_route_planted_tie_rule_flip_is_caught(orc):
    """Planted mistake: break ties toward the HIGHER id (negate the expert order
    by reversing columns) -- the tie-heavy golden must then disagree."""
    g = load("route_ties_t128")
    T, H, E, k, norm = (int(v) for v in g["meta"])
    rev_ids, _ = orc.route_from_logits(np.ascontiguousarray(g["logits"][:, ::-1]), k, True)
    flipped = (E - 1) - rev_ids
    assert not np.array_equal(flipped, g["ids"])


def test_route_planted_dropped_renorm_is_caught(orc):
    g = load("route_qwen_t64")
    _, w = orc.route_from_logits(g["logits"], 8, False)
    assert (ulp_diff_bf16(w, g["weights"]) > 1).mean() > 0.9


def test_route_tie_rule_brute_force(orc):
    rng = np.random.default_rng(4)
    for trial in range(300):
        E = int(rng.integers(2, 140))
        k = int(rng.integers(1, min(E, 9) + 1))
        T = 3
        levels = rng.integers(0, 4, (T, E)).astype(np.float32) * 0.25 - 0.5  # heavy ties
        logits = orc.f32_to_bf16(levels)
        ids, w, probs = orc.route_from_logits(logits, k, True, want_probs=True)
        for t in range(T):
            want = sorted(range(E), key=lambda e: (-probs[t, e], e))[:k]
            assert list(ids[t]) == want


def test_route_probs_closed_form(orc):
    rng = np.random.default_rng(5)
    logits = orc.f32_to_bf16(rng.standard_normal((32, 128)).astype(np.float32))
    _, _, probs = orc.route_from_logits(logits, 8, True, want_probs=True)
    l = orc.bf16_to_f32(logits).astype(np.float64)
    ref = np.exp(l - l.max(1, keepdims=True))
    ref /= ref.sum(1, keepdims=True)
    assert np.abs(probs - ref).max() / ref.max() < 1e-6
    assert np.allclose(probs.sum(1), 1.0, atol=1e-5)


def test_route_hist_is_bincount(orc):
    rng = np.random.default_rng(6)
    ids = rng.integers(0, 128, (100, 8)).astype(np.int32)
    assert np.array_equal(orc.route_hist(ids, 128), np.bincount(ids.reshape(-1), minlength=128))


# ------------------------------------------------------------------ pack

@pytest.mark.parametrize("name", ROUTE_CASES)
def test_pack_matches_both_reference_groupings(orc, name):
    g = load(f"route_{name}")
    T, H, E, k, norm = (int(v) for v in g["meta"])
    p = orc.pack(g["ids"], E)
    assert np.array_equal(p["counts"], g["counts"])
    assert np.array_equal(p["perm_token"], g["perm_token"])        # compact_expert_groups
    assert np.array_equal(p["perm_pos"], g["perm_pos"])
    assert np.array_equal(p["perm_token"], g["groups_token"])      # expert_groups (torch.where)
    assert np.array_equal(p["perm_pos"], g["groups_pos"])


def test_pack_planted_token_major_order_is_caught(orc):
    """Planted mistake: token-major (t*k+s) instead of slot-major flat order."""
    g = load("route_qwen_t64")
    T, k = g["ids"].shape
    wrong = orc.pack(np.ascontiguousarray(g["ids"].reshape(k, T)), 128)  # transposed operand
    assert not np.array_equal(wrong["perm_pos"], g["perm_pos"])


def test_pack_invariants_brute_force(orc):
    rng = np.random.default_rng(7)
    for trial in range(200):
        T = int(rng.integers(1, 300))
        k = int(rng.integers(1, 9))
        E = int(rng.integers(k, 200))
        ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
        p = orc.pack(ids, E)
        n = T * k
        assert p["offsets"][0] == 0 and p["offsets"][-1] == n
        assert np.array_equal(np.diff(p["offsets"]), p["counts"])
        assert np.array_equal(np.sort(p["perm_pos"]), np.arange(n))          # bijection
        assert np.array_equal(p["row_of"][p["perm_pos"]], np.arange(n))      # inverse map
        flat = ids.T.reshape(-1)                                             # slot-major
        want = sorted(range(n), key=lambda f: (flat[f], f))
        assert np.array_equal(p["perm_token"], np.array(want) % T)
        assert np.array_equal(p["perm_pos"], (np.array(want) % T) * k + np.array(want) // T)


def test_pack_rejects_out_of_range(orc):
    with pytest.raises(ValueError):
        orc.pack(np.array([[0, 200]], np.int32), 128)


# ------------------------------------------------------------------ expert

@pytest.mark.parametrize("name", ["small", "h2048_m4"])
def test_expert_forward_vs_torch(orc, name):
    g = load(f"expert_{name}")
    I, H = g["wg"].shape
    x = g["x"].reshape(-1, H)
    y = orc.expert_forward(x, g["wg"], g["wu"], g["wd"])
    ref = orc.bf16_to_f32(g["y_bf16"]).reshape(y.shape)
    got = orc.bf16_to_f32(y)
    # bf16 chain vs bf16 chain: roundings coincide except where torch's fp32
    # accumulation lands on the other side of a rounding boundary
    assert np.abs(got - ref).max() / np.abs(ref).max() < 1e-2
    assert ulp_diff_bf16(y, g["y_bf16"].reshape(y.shape)).max() <= 2
    yfp = orc.expert_forward_fp(x, g["wg"], g["wu"], g["wd"])
    assert np.abs(yfp - g["y_fp32"]).max() / np.abs(g["y_fp32"]).max() < 1e-5
    rel_l2 = np.linalg.norm(got - g["y_fp32"]) / np.linalg.norm(g["y_fp32"])
    assert rel_l2 < 0.02                      # pdscope_compare.py:692-695 bound


def test_expert_planted_swapped_projections_is_caught(orc):
    g = load("expert_small")
    I, H = g["wg"].shape
    y = orc.expert_forward(g["x"].reshape(-1, H), g["wu"], g["wg"], g["wd"])  # gate<->up swapped
    ref = orc.bf16_to_f32(g["y_bf16"]).reshape(y.shape)
    assert np.abs(orc.bf16_to_f32(y) - ref).max() / np.abs(ref).max() > 0.05


# ------------------------------------------------------------------ merge

def test_merge_closed_form(orc):
    rng = np.random.default_rng(8)
    T, k, H = 37, 8, 96
    y = orc.f32_to_bf16(rng.standard_normal((T * k, H)).astype(np.float32))
    w = orc.f32_to_bf16(rng.random((T, k)).astype(np.float32))
    row_of = rng.permutation(T * k).astype(np.int32)
    out = orc.merge(y, row_of, w)
    yf = orc.bf16_to_f32(y).astype(np.float64)
    wf = orc.bf16_to_f32(w).astype(np.float64)
    ref = np.einsum("tk,tkh->th", wf, yf[row_of.reshape(T, k)])
    want = np.array([orc.f64_to_bf16_scalar(v) for v in ref.reshape(-1)], np.uint16).reshape(T, H)
    assert np.array_equal(out, want)
    add = orc.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32))
    out2 = orc.merge(y, row_of, w, add_in=add)
    ref2 = ref + orc.bf16_to_f32(add)
    assert ulp_diff_bf16(out2, orc.f32_to_bf16(ref2.astype(np.float32))).max() <= 1


def test_merge_planted_row_map_is_caught(orc):
    rng = np.random.default_rng(9)
    T, k, H = 8, 4, 32
    y = orc.f32_to_bf16(rng.standard_normal((T * k, H)).astype(np.float32))
    w = orc.f32_to_bf16(rng.random((T, k)).astype(np.float32))
    row_of = rng.permutation(T * k).astype(np.int32)
    inverse = np.argsort(row_of).astype(np.int32)          # perm_pos used where row_of belongs
    assert not np.array_equal(orc.merge(y, row_of, w), orc.merge(y, inverse, w))


# ------------------------------------------------------------------ layer / CPU baseline

def _layer(rng, T, H, I, E):
    gate = orc_f32(rng.standard_normal((E, H)) * 0.02)
    slots = [orc_f32(rng.standard_normal(3 * I * H) * 0.02) for _ in range(E)]
    x = orc_f32(rng.standard_normal((T, H)))
    return x, gate, slots


def orc_f32(a):
    from oracle.oracle import f32_to_bf16
    return f32_to_bf16(np.asarray(a, np.float32))


def test_moe_layer_composes_the_pieces(orc):
    rng = np.random.default_rng(10)
    T, H, I, E, k = 6, 128, 64, 16, 4
    x, gate, slots = _layer(rng, T, H, I, E)
    res = orc.moe_layer(x, gate, slots, k)
    logits, ids, w = orc.route(x, gate, k)
    assert np.array_equal(res["ids"], ids) and np.array_equal(res["weights"], w)
    # per-token direct evaluation, no grouping
    for t in range(T):
        acc = np.zeros(H)
        for s in range(k):
            e = ids[t, s]
            blk = slots[e]
            yv = orc.expert_forward(x[t:t + 1], blk[:I * H].reshape(I, H), blk[I * H:2 * I * H].reshape(I, H),
                                    blk[2 * I * H:].reshape(H, I))
            acc += orc.bf16_to_f32(w[t:t + 1, s]).astype(np.float64)[0] * orc.bf16_to_f32(yv)[0]
        want = np.array([orc.f64_to_bf16_scalar(v) for v in acc], np.uint16)
        assert np.array_equal(res["out"][t], want)


def test_cpu_baseline_kernel_matches_oracle(orc):
    rng = np.random.default_rng(11)
    T, H, I, E, k = 3, 256, 128, 8, 4
    x, gate, slots = _layer(rng, T, H, I, E)
    ptrs = [s.ctypes.data for s in slots]
    logits, ids, w = orc.route(x, gate, k)
    out = orc.cpu_moe_decode(x[0], ids[0], w[0], ptrs, H, I, 4)
    ref = orc.moe_layer(x[:1], gate, slots, k)["out"][0]
    a, b = orc.bf16_to_f32(out), orc.bf16_to_f32(ref)
    assert np.abs(a - b).max() / np.abs(b).max() < 1e-2
    rows = orc.cpu_moe_rows(np.repeat(x[:1], k, 0), ids[0].astype(np.int64),
                            orc.bf16_to_f32(w[0]), ptrs, H, I, 4)
    merged = (orc.bf16_to_f32(rows).astype(np.float64)).sum(0)
    assert np.abs(merged - b).max() / np.abs(b).max() < 2e-2


# ------------------------------------------------------------------ reference-order merge / native tail

def test_merge_ordered_matches_torch_per_expert_index_add(orc):
    """merge='reference' (pdscope_runtime.py:454-468): the torch-CPU fixture adds
    each expert's weighted rows with index_add_ in ascending expert id; the
    oracle's per-token restatement must equal it bit for bit, and so must the
    row-by-row index_add over the grouped rows."""
    d = np.load(GOLDEN / "merge_t48.npz")
    ids, w, y, want = d["ids"], d["weights"], d["y"], d["out"]
    T, k = ids.shape
    p = orc.pack(ids, 32)
    assert np.array_equal(orc.merge_ordered(y, p["row_of"], w), want)
    rows_w = w.reshape(-1)[p["perm_pos"]]
    got = orc.index_add_bf16(np.zeros_like(want), p["perm_token"], y, rows_w)
    assert np.array_equal(got, want)


def test_merge_ordered_planted_mistakes_are_caught(orc):
    d = np.load(GOLDEN / "merge_t48.npz")
    ids, w, y, want = d["ids"], d["weights"], d["y"], d["out"]
    p = orc.pack(ids, 32)
    # one rounding in fp32 instead of bf16 sequential adds
    assert not np.array_equal(orc.merge(y, p["row_of"], w), want)
    # descending instead of ascending expert order
    rows_w = w.reshape(-1)[p["perm_pos"]]
    rev = np.arange(y.shape[0])[::-1].copy()
    got = orc.index_add_bf16(np.zeros_like(want), p["perm_token"][rev], y[rev], rows_w[rev])
    assert not np.array_equal(got, want)


def test_index_add_bf16_matches_native_tail_fixture(orc):
    """native_layer_dispatch.cpp:88: out.index_add_(0, tokens, scratch * weights[:, None]).
    Decode group (every row adds into token 0): each add rounded to bf16, rows
    in order; a group of distinct tokens: one add per token."""
    d = np.load(GOLDEN / "native_tail_r6.npz")
    rows = d["scratch"].shape[0]
    got = orc.index_add_bf16(d["out0"][:1], np.zeros(rows, np.int64), d["scratch"], d["weights"])
    assert np.array_equal(got, d["out_decode"])
    got = orc.index_add_bf16(d["out0"], d["tokens"], d["scratch"], d["weights"])
    assert np.array_equal(got, d["out_distinct"])
    # a single row reduces to one bf16 product and one bf16 sum
    one = orc.index_add_bf16(d["out0"][:1], np.zeros(1, np.int64), d["scratch"][:1], d["weights"][:1])
    prod = orc.f32_to_bf16(orc.bf16_to_f32(d["scratch"][0]) * orc.bf16_to_f32(d["weights"][:1])[0])
    assert np.array_equal(one[0], orc.f32_to_bf16(orc.bf16_to_f32(d["out0"][0]) + orc.bf16_to_f32(prod)))
    # planted: fp32 accumulation of the decode group's rows (one rounding) differs
    acc = orc.bf16_to_f32(d["out0"][0]).astype(np.float32)
    for r in range(rows):
        acc = acc + orc.bf16_to_f32(orc.f32_to_bf16(orc.bf16_to_f32(d["scratch"][r]) *
                                                    orc.bf16_to_f32(d["weights"][r:r + 1])[0]))
    assert not np.array_equal(orc.f32_to_bf16(acc), d["out_decode"][0])
