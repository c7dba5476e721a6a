"""GPU parity tests: every kernel through the C-ABI against the oracle.

Routing ids, weights and probabilities must be bit-exact with the oracle
applied to the kernel's own bf16 logits (the logits themselves are checked
against the exactly rounded dot products within fp32 accumulation error).
Grouping (counts, offsets, permutations, inverse map) must be bit-exact.
Expert outputs and the merged layer must be within max rel err <= 1e-2 and
mean abs err <= 1e-3 of the oracle's bf16 expert path.
"""
import numpy as np
import pytest
import torch

from tests.gpu_helpers import (MAX_REL, MEAN_ABS, err_metrics, from_u16, logits_within_accumulation_error, u16,
                               ulp_diff_bf16)

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module")
def pd():
    from pdscope_amd import ops, layer, synthetic
    return ops, layer, synthetic


@pytest.fixture(scope="module")
def qwen(pd):
    _, _, synthetic = pd
    lay = synthetic.make_layer(**{k: v for k, v in synthetic.QWEN.items()}, device=DEV)
    torch.cuda.synchronize()
    return lay


@pytest.fixture(scope="module")
def qwen_host(qwen):
    return dict(gate=u16(qwen.gate), experts=u16(qwen.experts))


def _route_check(orc, ops, x, gate, k, normalize, bias=None):
    logits, ids, w, probs = ops.route_topk(x, gate, k, normalize, bias=bias, capture_probabilities=True)
    torch.cuda.synchronize()
    lk, ik, wk, pk = u16(logits), ids.cpu().numpy(), u16(w), probs.cpu().numpy()
    bias_np = None if bias is None else bias.cpu().numpy()
    oi, ow, op = orc.route_from_logits(lk, k, normalize, bias_np, want_probs=True)
    assert np.array_equal(ik, oi), "top-k ids differ from the oracle given identical logits"
    assert np.array_equal(wk, ow), "routing weights differ from the oracle given identical logits"
    assert np.array_equal(pk.view(np.uint32), op.view(np.uint32)), "softmax probabilities not bit-exact"
    exact = orc.route_logits(u16(x), u16(gate))
    ok, nmis = logits_within_accumulation_error(lk, exact, u16(x), u16(gate), orc.bf16_to_f32)
    assert ok, "logit mismatch beyond fp32 accumulation error"
    assert nmis <= max(2, 2e-3 * lk.size), f"{nmis} logit mismatches"
    return lk, ik, wk


@pytest.mark.parametrize("T", [1, 2, 5, 8])
def test_route_small_T_qwen(orc, pd, qwen, T):
    ops, _, synthetic = pd
    x = synthetic.make_tokens(T, 2048, seed=100 + T)
    _route_check(orc, ops, x, qwen.gate, 8, True)


@pytest.mark.parametrize("T", [9, 33, 512, 2100, 4096])
def test_route_mfma_qwen(orc, pd, qwen, T):
    ops, _, synthetic = pd
    x = synthetic.make_tokens(T, 2048, seed=200 + T)
    _route_check(orc, ops, x, qwen.gate, 8, True)


@pytest.mark.parametrize("T", [1, 4096])
def test_route_zipf_bias(orc, pd, qwen, T):
    ops, _, synthetic = pd
    x = synthetic.make_tokens(T, 2048, seed=300 + T)
    bias, _ = synthetic.zipf_bias(128, device=DEV)
    _, ids, _ = _route_check(orc, ops, x, qwen.gate, 8, True, bias=bias)
    if T > 1:
        counts = np.bincount(ids.reshape(-1), minlength=128)
        assert counts.max() > 4 * counts.mean()  # skew reached the routing


@pytest.mark.parametrize("T", [1, 48, 1304])
def test_route_deepseek_no_renorm(orc, pd, T):
    ops, _, synthetic = pd
    gen = torch.Generator(device=DEV).manual_seed(7)
    gate = (torch.randn((64, 2048), generator=gen, device=DEV) * 0.02).to(torch.bfloat16)
    x = synthetic.make_tokens(T, 2048, seed=400 + T)
    _route_check(orc, ops, x, gate, 6, False)


@pytest.mark.parametrize("T", [3, 100])
def test_route_256_experts_top16(orc, pd, T):
    ops, _, synthetic = pd
    gen = torch.Generator(device=DEV).manual_seed(9)
    gate = (torch.randn((256, 1024), generator=gen, device=DEV) * 0.02).to(torch.bfloat16)
    x = synthetic.make_tokens(T, 1024, seed=450 + T)
    _route_check(orc, ops, x, gate, 16, True)


@pytest.mark.parametrize("T", [1, 64])
def test_route_tie_heavy(orc, pd, T):
    """Few distinct router rows and coarse activations: many exact logit ties."""
    ops, _, _ = pd
    gen = torch.Generator(device=DEV).manual_seed(11)
    rows = (torch.randn((4, 256), generator=gen, device=DEV) * 0.02).to(torch.bfloat16)
    gate = rows[torch.randint(0, 4, (128,), generator=gen, device=DEV)].contiguous()
    x = (torch.randint(-2, 3, (T, 256), generator=gen, device=DEV).float() * 0.5).to(torch.bfloat16)
    lk, ik, _ = _route_check(orc, ops, x, gate, 8, True)
    # ties were really exercised: some token has equal logits across its 8/9 boundary
    srt = np.sort(orc.bf16_to_f32(lk), axis=1)[:, ::-1]
    assert (srt[:, 7] == srt[:, 8]).any()


@pytest.mark.parametrize("T", [1, 64])
def test_route_probability_collisions(orc, pd, T):
    """Distinct logits whose probabilities underflow to the same value (0):
    three experts carry the mass, the other five of the top 8 are chosen
    among equal probabilities by lower id, while the logits rank those
    experts the other way (higher ids have the larger logits)."""
    ops, _, _ = pd
    gen = torch.Generator(device=DEV).manual_seed(13)
    E, H = 128, 256
    scale = -1.0 - (E - 1 - torch.arange(E, device=DEV, dtype=torch.float32)) * 0.01
    scale[[100, 50, 7]] = torch.tensor([0.01, 0.005, 0.0], device=DEV)
    gate = scale[:, None].expand(E, H).to(torch.bfloat16).contiguous()
    x = (torch.rand((T, H), generator=gen, device=DEV) + 0.5).to(torch.bfloat16)
    _, ik, _ = _route_check(orc, ops, x, gate, 8, True)
    assert (ik[:, :3] == [100, 50, 7]).all() and (ik[:, 3:] == [0, 1, 2, 3, 4]).all()


@pytest.mark.parametrize("E,k", [(64, 6), (128, 8), (256, 16)])
def test_route_staged_partials_equal_unstaged(pd, E, k):
    """From 2048 tokens the partial logits come from the LDS-staged kernel
    (128 tokens per block); below, from the 32-token kernel.  Both add the
    same MFMA chains, so the first 2047 tokens route bit for bit alike."""
    ops, _, synthetic = pd
    gen = torch.Generator(device=DEV).manual_seed(17 + E)
    gate = (torch.randn((E, 2048), generator=gen, device=DEV) * 0.02).to(torch.bfloat16)
    x = synthetic.make_tokens(2048, 2048, seed=500 + E)
    la, ia, wa, _ = ops.route_topk(x, gate, k, True)
    lb, ib, wb, _ = ops.route_topk(x[:2047].contiguous(), gate, k, True)
    torch.cuda.synchronize()
    assert torch.equal(la[:2047].view(torch.int16), lb.view(torch.int16))
    assert torch.equal(ia[:2047], ib) and torch.equal(wa[:2047].view(torch.int16), wb.view(torch.int16))


def test_route_hist(orc, pd):
    ops, _, _ = pd
    ids = torch.randint(0, 128, (4096, 8), device=DEV, dtype=torch.int32)
    hist = ops.route_hist(ids, 128)
    assert np.array_equal(hist.cpu().numpy(), orc.route_hist(ids.cpu().numpy(), 128))


def test_route_rejects_bad_args(pd, qwen):
    ops, _, synthetic = pd
    x = synthetic.make_tokens(2, 2048)
    with pytest.raises(ValueError):
        ops.route_topk(x, qwen.gate, 0, True)
    with pytest.raises(ValueError):
        ops.route_topk(x.float(), qwen.gate, 8, True)


# ------------------------------------------------------------------ pack

def _pack_check(orc, ops, ids_np, E):
    ids = torch.from_numpy(ids_np.astype(np.int32)).to(DEV)
    p = ops.pack(ids, E)
    torch.cuda.synchronize()
    o = orc.pack(ids_np, E)
    for name in ("counts", "offsets", "perm_token", "perm_pos", "row_of"):
        assert np.array_equal(getattr(p, name).cpu().numpy(), o[name]), name


@pytest.mark.parametrize("T,k,E", [(1, 8, 128), (7, 8, 128), (512, 8, 128), (4096, 8, 128), (1304, 6, 64),
                                   (3, 1, 32), (1000, 16, 256), (4099, 8, 128), (20000, 6, 64), (16384, 8, 128)])
def test_pack_uniform(orc, pd, T, k, E):
    ops, _, _ = pd
    rng = np.random.default_rng(T * 31 + k)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)])
    _pack_check(orc, ops, ids, E)


def test_pack_zipf_skew(orc, pd):
    ops, _, _ = pd
    rng = np.random.default_rng(5)
    p = np.arange(1, 129, dtype=np.float64) ** -1.1
    p /= p.sum()
    ids = np.stack([rng.choice(128, 8, replace=False, p=p) for _ in range(4096)])
    _pack_check(orc, ops, ids, 128)


def test_pack_all_one_expert_column(orc, pd):
    """Every token routes slot 0 to expert 0: one run of T rows, many empty experts."""
    ops, _, _ = pd
    T, k = 3000, 4
    ids = np.stack([np.array([0, 1 + (t % 3), 10, 20 + (t % 7)]) for t in range(T)])
    _pack_check(orc, ops, ids, 128)


# ------------------------------------------------------------------ experts

def _oracle_layer_given_routing(orc, x_u16, ids, w_u16, experts_u16, H, I):
    """Oracle expert path + merge for a given routing (ids/weights)."""
    E = experts_u16.shape[0]
    p = orc.pack(ids, E)
    xg = x_u16[p["perm_token"]]
    y = np.empty((ids.size, H), np.uint16)
    IH = I * H
    for e in np.nonzero(p["counts"])[0]:
        a, b = p["offsets"][e], p["offsets"][e + 1]
        blk = experts_u16[e]
        y[a:b] = orc.expert_forward(xg[a:b], blk[:IH].reshape(I, H), blk[IH:2 * IH].reshape(I, H),
                                    blk[2 * IH:].reshape(H, I))
    return orc.merge(y, p["row_of"], w_u16), y, p


@pytest.mark.parametrize("T", [2, 16, 64])
def test_layer_prefill_qwen(orc, pd, qwen, qwen_host, T):
    ops, layer, synthetic = pd
    x = synthetic.make_tokens(T, 2048, seed=500 + T)
    ws = layer.MoEWorkspace(T, 2048, 768, 128, 8, DEV)
    slots = ops.slot_table([qwen.experts[e] for e in range(128)], DEV)
    out, logits, ids, w = layer.moe_forward(x, qwen.gate, slots, ws)
    torch.cuda.synchronize()
    xu, ik, wk = u16(x), ids.cpu().numpy(), u16(w)
    oi, ow = orc.route_from_logits(u16(logits), 8, True)
    assert np.array_equal(ik, oi) and np.array_equal(wk, ow)
    ref, y_ref, p = _oracle_layer_given_routing(orc, xu, ik, wk, qwen_host["experts"], 2048, 768)
    # per-row expert outputs (grouped order) before the merge
    y_k = u16(ws.y[:T * 8 * 2048]).reshape(T * 8, 2048)
    m_y = err_metrics(orc.bf16_to_f32(y_k), orc.bf16_to_f32(y_ref))
    assert m_y["max_rel"] <= MAX_REL and m_y["mean_abs"] <= MEAN_ABS, m_y
    m = err_metrics(orc.bf16_to_f32(u16(out)), orc.bf16_to_f32(ref))
    assert m["max_rel"] <= MAX_REL and m["mean_abs"] <= MEAN_ABS, m


def test_layer_prefill_qwen_t4096_sampled_tokens(orc, pd, qwen, qwen_host):
    """The full T=4096 layer (the 384-row tile the workload uses, all 128
    experts, every tile boundary) checked on a seeded sample of tokens: for
    each sampled token its k grouped rows (ws.y, located through the device
    row map) against the oracle's expert outputs for that token, and its
    merged output against the oracle merge of those rows.  The grouping
    itself is checked bit-exact in full."""
    ops, layer, synthetic = pd
    T, H, I, k = 4096, 2048, 768, 8
    x = synthetic.make_tokens(T, H, seed=4096)
    ws = layer.MoEWorkspace(T, H, I, 128, k, DEV)
    slots = ops.slot_table([qwen.experts[e] for e in range(128)], DEV)
    out, logits, ids, w = layer.moe_forward(x, qwen.gate, slots, ws)
    torch.cuda.synchronize()
    assert ops.grouped_block_m(T * k // 128, int(ws.counts.max())) == 384
    ik, wk, xu = ids.cpu().numpy(), u16(w), u16(x)
    oi, ow = orc.route_from_logits(u16(logits), k, True)
    assert np.array_equal(ik, oi) and np.array_equal(wk, ow)
    p = orc.pack(np.ascontiguousarray(ik, dtype=np.int32), 128)
    assert np.array_equal(ws.row_of[:T * k].cpu().numpy(), p["row_of"])
    rng = np.random.default_rng(4096)
    tokens = np.sort(rng.choice(T, 40, replace=False))
    tokens[0], tokens[-1] = 0, T - 1
    IH = I * H
    y_all = u16(ws.y[:T * k * H]).reshape(T * k, H)
    row_of = p["row_of"].reshape(T, k)
    got_y, ref_y = [], []
    for t in tokens:
        for s in range(k):
            blk = qwen_host["experts"][ik[t, s]]
            ref_y.append(orc.expert_forward(xu[t:t + 1], blk[:IH].reshape(I, H), blk[IH:2 * IH].reshape(I, H),
                                            blk[2 * IH:].reshape(H, I))[0])
            got_y.append(y_all[row_of[t, s]])
    got_y, ref_y = np.stack(got_y), np.stack(ref_y)
    m_y = err_metrics(orc.bf16_to_f32(got_y), orc.bf16_to_f32(ref_y))
    assert m_y["max_rel"] <= MAX_REL and m_y["mean_abs"] <= MEAN_ABS, m_y
    # merge of the sampled tokens' device rows, in slot order
    local_row_of = np.arange(len(tokens) * k, dtype=np.int32).reshape(len(tokens), k)
    ref_out = orc.merge(got_y, local_row_of, wk[tokens])
    d = ulp_diff_bf16(u16(out)[tokens], ref_out)
    assert (d <= 1).all() and (d > 0).mean() < 1e-3, "merge of the sampled tokens differs from the oracle merge"


@pytest.mark.parametrize("bm", [32, 64, 128, 256, 384])
def test_grouped_block_m_variants(orc, pd, bm):
    """Every row tile on a small layer with ragged expert sizes (0..many rows)."""
    ops, layer, synthetic = pd
    H, I, E, k, T = 256, 128, 32, 4, 150
    lay = synthetic.make_layer(H, I, E, k, True, seed=900 + bm, device=DEV)
    x = synthetic.make_tokens(T, H, seed=901 + bm)
    ws = layer.MoEWorkspace(T, H, I, E, k, DEV)
    slots = ops.slot_table([lay.experts[e] for e in range(E)], DEV)
    # skew: bias the router so a few experts get most rows
    bias = torch.zeros(E, device=DEV)
    bias[3] = 4.0
    bias[7] = 2.0
    out, logits, ids, w = layer.moe_forward(x, lay.gate, slots, ws, bias=bias, block_m=bm)
    torch.cuda.synchronize()
    ik, wk = ids.cpu().numpy(), u16(w)
    ref, _, p = _oracle_layer_given_routing(orc, u16(x), ik, wk, u16(lay.experts), H, I)
    assert p["counts"].max() >= 100  # one expert holds most tokens: many row tiles
    m = err_metrics(orc.bf16_to_f32(u16(out)), orc.bf16_to_f32(ref))
    assert m["max_rel"] <= MAX_REL and m["mean_abs"] <= MEAN_ABS, m


@pytest.mark.parametrize("bm", [128, 256, 384])
def test_grouped_qwen_multi_tile_experts(orc, pd, qwen, qwen_host, bm):
    """Qwen shape with a skewed router: hot experts span several row tiles
    (and the weight tiles they share), cold ones a partial tile or none."""
    ops, layer, synthetic = pd
    T = 600
    x = synthetic.make_tokens(T, 2048, seed=950 + bm)
    ws = layer.MoEWorkspace(T, 2048, 768, 128, 8, DEV)
    slots = ops.slot_table([qwen.experts[e] for e in range(128)], DEV)
    bias = torch.zeros(128, device=DEV)
    bias[5], bias[77], bias[100] = 6.0, 5.0, 4.0
    out, logits, ids, w = layer.moe_forward(x, qwen.gate, slots, ws, bias=bias, block_m=bm)
    torch.cuda.synchronize()
    ik, wk = ids.cpu().numpy(), u16(w)
    ref, y_ref, p = _oracle_layer_given_routing(orc, u16(x), ik, wk, qwen_host["experts"], 2048, 768)
    assert p["counts"].max() > 2 * bm // 2
    y_k = u16(ws.y[:T * 8 * 2048]).reshape(T * 8, 2048)
    m_y = err_metrics(orc.bf16_to_f32(y_k), orc.bf16_to_f32(y_ref))
    assert m_y["max_rel"] <= MAX_REL and m_y["mean_abs"] <= MEAN_ABS, m_y
    m = err_metrics(orc.bf16_to_f32(u16(out)), orc.bf16_to_f32(ref))
    assert m["max_rel"] <= MAX_REL and m["mean_abs"] <= MEAN_ABS, m


def _snake_order(rows, sel):
    """Restatement of the balanced order: rank by rows (descending, ties by
    position), deal rank r to group r%8 (even rounds) or 7-r%8 (odd rounds),
    concatenate the groups."""
    ranked = sorted(range(len(sel)), key=lambda i: (-rows[sel[i]], i))
    groups = [[] for _ in range(8)]
    for r, i in enumerate(ranked):
        groups[r % 8 if (r // 8) % 2 == 0 else 7 - r % 8].append(sel[i])
    return [e for g in groups for e in g]


@pytest.mark.parametrize("nsel,bm", [(128, 256), (61, 64), (7, 128), (1, 32), (256, 64)])
def test_schedule_balanced_order_and_same_outputs(pd, nsel, bm):
    """The balanced order is the snake deal of the size ranking, tile_start is
    its m-tile prefix, and the grouped outputs do not depend on the order
    (bitwise: every row is computed by the same tile arithmetic)."""
    ops, layer, synthetic = pd
    g = torch.Generator().manual_seed(nsel * 31 + bm)
    E = max(nsel, 8)
    H, I = 256, 128
    rows = (torch.rand(E, generator=g) ** 3 * 300).to(torch.int32)
    rows[torch.randperm(E, generator=g)[:E // 5]] = 17  # ties
    sel_list = sorted(torch.randperm(E, generator=g)[:nsel].tolist())
    counts = rows.to(DEV)
    offsets = torch.zeros(E + 1, dtype=torch.int32)
    offsets[1:] = torch.cumsum(rows, 0)
    n = int(offsets[-1])
    sel = torch.tensor(sel_list, dtype=torch.int32, device=DEV)
    order = torch.empty(nsel, dtype=torch.int32, device=DEV)
    ts = ops.schedule(counts, sel, bm, order=order)
    torch.cuda.synchronize()
    want = _snake_order(rows.tolist(), sel_list)
    assert order.cpu().tolist() == want
    tiles = [(int(rows[e]) + bm - 1) // bm for e in want]
    assert ts.cpu().tolist() == [0] + np.cumsum(tiles).tolist()
    # same outputs as the identity order
    lay = synthetic.make_layer(H, I, E, 4, True, seed=nsel + bm, device=DEV)
    slots = ops.slot_table([lay.experts[e] for e in range(E)], DEV)
    x = synthetic.make_tokens(max(n, 1), H, seed=bm)
    perm = torch.randint(0, max(n, 1), (max(n, 1),), generator=g, dtype=torch.int32).to(DEV)
    off_d = offsets.to(DEV)
    outs = []
    for s_, t_ in ((sel, ops.schedule(counts, sel, bm)), (order, ts)):
        h = torch.zeros(max(n, 1) * I, dtype=torch.bfloat16, device=DEV)
        y = torch.zeros((max(n, 1), H), dtype=torch.bfloat16, device=DEV)
        mt = (n + bm - 1) // bm + nsel
        ops.swiglu_grouped(x, perm, off_d, s_, t_, mt, bm, slots, H, I, h, y)
        outs.append((h, y))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("nsel,bm,bm2", [(128, 384, 256), (61, 64, 128), (1, 32, 384), (256, 256, 32)])
def test_schedule_balanced_pair_equals_two_schedules(pd, nsel, bm, bm2):
    """The paired launch writes the order and both tile prefixes of two
    separate balanced schedules, and the gate/up + down launches over them
    equal the one-tile grouped launch (bitwise)."""
    ops, layer, synthetic = pd
    g = torch.Generator().manual_seed(nsel * 7 + bm2)
    E = max(nsel, 8)
    rows = (torch.rand(E, generator=g) ** 3 * 700).to(torch.int32)
    rows[torch.randperm(E, generator=g)[:E // 4]] = 0
    sel = torch.tensor(sorted(torch.randperm(E, generator=g)[:nsel].tolist()), dtype=torch.int32, device=DEV)
    counts = rows.to(DEV)
    order1, order2 = (torch.full((nsel,), -1, dtype=torch.int32, device=DEV) for _ in range(2))
    ts1 = ops.schedule(counts, sel, bm, order=order1)
    ts2 = ops.schedule(counts, sel, bm2, order=order2)
    order = torch.full((nsel,), -1, dtype=torch.int32, device=DEV)
    out1, out2 = (torch.full((nsel + 1,), -1, dtype=torch.int32, device=DEV) for _ in range(2))
    ops.schedule(counts, sel, bm, out=out1, order=order, block_m2=bm2, out2=out2)
    torch.cuda.synchronize()
    assert torch.equal(order, order1) and torch.equal(order, order2)
    assert torch.equal(out1, ts1) and torch.equal(out2, ts2)
    with pytest.raises(ValueError):
        ops.schedule(counts, sel, bm, out=out1, block_m2=bm2, out2=out2)


@pytest.mark.parametrize("T,k,E,nsel,bm,bm2", [(5, 8, 128, 128, 64, 0), (256, 8, 128, 128, 64, 0),
                                                (512, 8, 128, 128, 64, 0), (4096, 8, 128, 128, 384, 256),
                                                (1304, 6, 64, 40, 128, 0), (3000, 8, 256, 256, 256, 32),
                                                (700, 4, 32, 17, 32, 384)])
def test_pack_with_schedule_equals_pack_then_schedule(pd, T, k, E, nsel, bm, bm2):
    """pdscope_pack_schedule_balanced: the grouping bit-exact with
    pdscope_pack and the order / tile prefixes with pdscope_schedule_balanced
    (_pair) over the counts it produced, on the single-block (T*k <= 2048)
    and multi-block paths, over all experts and over subsets."""
    ops, layer, synthetic = pd
    g = torch.Generator().manual_seed(T * 7 + E + nsel)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32).to(DEV)
    sel = torch.tensor(sorted(torch.randperm(E, generator=g)[:nsel].tolist()), dtype=torch.int32, device=DEV)
    ref = ops.pack(ids, E)
    o1 = torch.empty(nsel, dtype=torch.int32, device=DEV)
    t1 = torch.empty(nsel + 1, dtype=torch.int32, device=DEV)
    t2 = torch.empty(nsel + 1, dtype=torch.int32, device=DEV)
    if bm2:
        ops.schedule(ref.counts, sel, bm, out=t1, order=o1, block_m2=bm2, out2=t2)
    else:
        ops.schedule(ref.counts, sel, bm, out=t1, order=o1)
    order = torch.full((nsel,), -1, dtype=torch.int32, device=DEV)
    ts = torch.full((nsel + 1,), -1, dtype=torch.int32, device=DEV)
    ts2 = torch.full((nsel + 1,), -1, dtype=torch.int32, device=DEV)
    got = ops.pack(ids, E, schedule=(sel, bm, order, ts) + ((bm2, ts2) if bm2 else ()))
    torch.cuda.synchronize()
    for name in ("counts", "offsets", "perm_token", "perm_pos", "row_of"):
        assert torch.equal(getattr(got, name), getattr(ref, name)), name
    assert torch.equal(order, o1) and torch.equal(ts, t1)
    if bm2:
        assert torch.equal(ts2, t2)


@pytest.mark.parametrize("T,k,E", [(40, 8, 128), (3000, 8, 64)])
def test_schedules_count_out_of_range_sel_entries_as_empty(pd, T, k, E):
    """A sel entry outside [0, E) (negative, E, past 256, INT32_MAX) is an
    expert with no rows in every schedule: pdscope_schedule, the balanced
    order and prefixes (one and two row tiles) and the schedule the pack
    launch writes (single- and multi-block).  It gets no tiles and ranks with
    the untouched experts, and nothing is read past `counts`."""
    from collections import defaultdict
    ops, layer, synthetic = pd
    g = torch.Generator().manual_seed(T + E)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32).to(DEV)
    sel_list = [3, E + 5, 7, -1, 11, 300, 2 ** 31 - 1, E, 0, E - 1]
    sel = torch.tensor(sel_list, dtype=torch.int32, device=DEV)
    n = len(sel_list)
    ref = ops.pack(ids, E)
    torch.cuda.synchronize()
    rows = defaultdict(int, enumerate(ref.counts.cpu().tolist()))
    bm, bm2 = 64, 256
    plain = ops.schedule(ref.counts, sel, bm)
    o1 = torch.empty(n, dtype=torch.int32, device=DEV)
    t1 = ops.schedule(ref.counts, sel, bm, order=o1)
    o2, t2, t2b = (torch.empty(n, dtype=torch.int32, device=DEV), torch.empty(n + 1, dtype=torch.int32, device=DEV),
                   torch.empty(n + 1, dtype=torch.int32, device=DEV))
    ops.schedule(ref.counts, sel, bm, out=t2, order=o2, block_m2=bm2, out2=t2b)
    o3, t3, t3b = (torch.full((n,), -7, dtype=torch.int32, device=DEV),
                   torch.full((n + 1,), -7, dtype=torch.int32, device=DEV),
                   torch.full((n + 1,), -7, dtype=torch.int32, device=DEV))
    got = ops.pack(ids, E, schedule=(sel, bm, o3, t3, bm2, t3b))
    torch.cuda.synchronize()
    for name in ("counts", "offsets", "perm_token", "row_of"):
        assert torch.equal(getattr(got, name), getattr(ref, name)), name
    tiles = lambda es, b: [0] + np.cumsum([(rows[e] + b - 1) // b for e in es]).tolist()  # noqa: E731
    assert plain.cpu().tolist() == tiles(sel_list, bm)
    want = _snake_order(rows, sel_list)
    for o, t in ((o1, t1), (o2, t2), (o3, t3)):
        assert o.cpu().tolist() == want and t.cpu().tolist() == tiles(want, bm)
    for t in (t2b, t3b):
        assert t.cpu().tolist() == tiles(want, bm2)


def test_decode_qwen(orc, pd, qwen, qwen_host):
    ops, layer, synthetic = pd
    ws = layer.MoEWorkspace(1, 2048, 768, 128, 8, DEV)
    slots = ops.slot_table([qwen.experts[e] for e in range(128)], DEV)
    for seed in (600, 601, 602):
        x = synthetic.make_tokens(1, 2048, seed=seed)
        out, logits, ids, w = layer.moe_forward(x, qwen.gate, slots, ws)
        torch.cuda.synchronize()
        ik, wk = ids.cpu().numpy(), u16(w)
        oi, ow = orc.route_from_logits(u16(logits), 8, True)
        assert np.array_equal(ik, oi) and np.array_equal(wk, ow)
        ref, _, _ = _oracle_layer_given_routing(orc, u16(x), ik, wk, qwen_host["experts"], 2048, 768)
        m = err_metrics(orc.bf16_to_f32(u16(out)), orc.bf16_to_f32(ref))
        assert m["max_rel"] <= MAX_REL and m["mean_abs"] <= MEAN_ABS, m


def test_decode_equals_grouped_path(orc, pd, qwen):
    """T=1 through K4 and through K2+K3+K5 (forced) agree within bf16 tolerance."""
    ops, layer, synthetic = pd
    x = synthetic.make_tokens(1, 2048, seed=700)
    ws = layer.MoEWorkspace(2, 2048, 768, 128, 8, DEV)
    slots = ops.slot_table([qwen.experts[e] for e in range(128)], DEV)
    logits, ids, w = layer.route(x, qwen.gate, ws)
    dec = layer.experts_resident(x, ids, w, slots, ws).clone()
    # grouped path on the same routing: duplicate the token and keep row 0
    x2 = torch.cat([x, x]).contiguous()
    ids2 = torch.cat([ids, ids]).contiguous()
    w2 = torch.cat([w, w]).contiguous()
    grp = layer.experts_resident(x2, ids2, w2, slots, ws)[:1].clone()
    torch.cuda.synchronize()
    m = err_metrics(orc.bf16_to_f32(u16(dec)), orc.bf16_to_f32(u16(grp)))
    assert m["max_rel"] <= MAX_REL and m["mean_abs"] <= MEAN_ABS, m


def test_merge_matches_oracle(orc, pd):
    ops, _, _ = pd
    rng = np.random.default_rng(12)
    T, k, H = 300, 8, 2048
    y = orc.f32_to_bf16(rng.standard_normal((T * k, H)).astype(np.float32) * 0.3)
    w = orc.f32_to_bf16(rng.random((T, k)).astype(np.float32) / k)
    row_of = rng.permutation(T * k).astype(np.int32)
    out = torch.empty((T, H), dtype=torch.bfloat16, device=DEV)
    ops.merge(from_u16(y), torch.from_numpy(row_of).to(DEV), from_u16(w), out)
    torch.cuda.synchronize()
    ref = orc.merge(y, row_of, w)
    d = ulp_diff_bf16(u16(out), ref)
    assert (d <= 1).all() and (d > 0).mean() < 1e-3
    add = orc.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32))
    ops.merge(from_u16(y), torch.from_numpy(row_of).to(DEV), from_u16(w), out, add_in=from_u16(add))
    torch.cuda.synchronize()
    m = err_metrics(orc.bf16_to_f32(u16(out)), orc.bf16_to_f32(orc.merge(y, row_of, w, add_in=add)))
    assert m["max_rel"] < 1e-2


@pytest.mark.parametrize("T,k", [(300, 8), (40, 6), (1500, 8), (200, 16)])
def test_merge_ordered_matches_oracle_bit_exact(orc, pd, T, k):
    """merge='reference': rows added in ascending grouped row (expert id) in
    bf16 arithmetic, bit-exact with the oracle, with and without the
    unweighted add_in (added last); T > 1024 runs the any-k loop."""
    ops, _, _ = pd
    rng = np.random.default_rng(13 + T + k)
    H = 2048
    y = orc.f32_to_bf16(rng.standard_normal((T * k, H)).astype(np.float32) * 0.3)
    w = orc.f32_to_bf16(rng.random((T, k)).astype(np.float32) / k)
    row_of = rng.permutation(T * k).astype(np.int32)
    add = orc.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32))
    out = torch.empty((T, H), dtype=torch.bfloat16, device=DEV)
    for add_in in (None, add):
        ops.merge(from_u16(y), torch.from_numpy(row_of).to(DEV), from_u16(w), out,
                  add_in=None if add_in is None else from_u16(add_in), mode="reference")
        torch.cuda.synchronize()
        assert np.array_equal(u16(out), orc.merge_ordered(y, row_of, w, add_in=add_in))


def test_stage_merge_matches_bf16_index_add(pd):
    ops, _, _ = pd
    rows, H = 8, 2048
    g = torch.Generator().manual_seed(3)
    block = torch.randn((rows, H), generator=g).to(torch.bfloat16).pin_memory()
    weights = torch.rand(rows, generator=g).to(torch.bfloat16).to(DEV)
    tokens = torch.zeros(rows, dtype=torch.int64, device=DEV)
    scratch = torch.empty((rows, H), dtype=torch.bfloat16, device=DEV)
    out = torch.zeros((1, H), dtype=torch.bfloat16, device=DEV)
    ops.stage_merge(block.data_ptr(), rows, H * 2, scratch, out, tokens, weights)
    torch.cuda.synchronize()
    # sequential bf16 restatement of out.index_add_(0, tokens, scratch * weights[:, None])
    ref = torch.zeros(H, dtype=torch.bfloat16)
    prod = (block * weights.cpu()[:, None])
    for r in range(rows):
        ref = (ref.float() + prod[r].float()).to(torch.bfloat16)
    assert torch.equal(out.cpu()[0], ref)
    assert torch.equal(scratch.cpu(), block)


def test_deepseek_v2_lite_layer_with_shared_experts(orc, pd):
    """DeepSeek-V2-Lite layer: 64 routed experts of 1408, top-6 without
    renormalisation, plus 2 shared experts (one 2816-wide MLP over every
    token, added unweighted in the merge).  Routing bit-exact given the
    logits; routed rows and the layer output within bf16 tolerance."""
    ops, layer, synthetic = pd
    cfg = dict(synthetic.DSV2)
    H, I, E, k, Is = cfg["H"], cfg["I"], cfg["E"], cfg["k"], cfg["shared_I"]
    lay = synthetic.make_layer(H, I, E, k, False, seed=321, device=DEV, shared_I=Is)
    T = 40
    x = synthetic.make_tokens(T, H, seed=322)
    ws = layer.MoEWorkspace(T, H, I, E, k, DEV, shared_I=Is)
    slots = ops.slot_table([lay.experts[e] for e in range(E)], DEV)
    shared_slot = ops.slot_table([lay.shared], DEV)
    out, logits, ids, w = layer.moe_forward(x, lay.gate, slots, ws, normalize=False, shared_slot=shared_slot)
    torch.cuda.synchronize()
    ik, wk = ids.cpu().numpy(), u16(w)
    oi, ow = orc.route_from_logits(u16(logits), k, False)
    assert np.array_equal(ik, oi) and np.array_equal(wk, ow)
    xu = u16(x)
    _, y_ref, p = _oracle_layer_given_routing(orc, xu, ik, wk, u16(lay.experts), H, I)
    sh = u16(lay.shared)
    IsH = Is * H
    shared_ref = orc.expert_forward(xu, sh[:IsH].reshape(Is, H), sh[IsH:2 * IsH].reshape(Is, H),
                                    sh[2 * IsH:].reshape(H, Is))
    m_s = err_metrics(orc.bf16_to_f32(u16(ws.y_shared[:T])), orc.bf16_to_f32(shared_ref))
    assert m_s["max_rel"] <= MAX_REL and m_s["mean_abs"] <= MEAN_ABS, m_s
    ref = orc.merge(y_ref, p["row_of"], wk, add_in=shared_ref)
    m = err_metrics(orc.bf16_to_f32(u16(out)), orc.bf16_to_f32(ref))
    assert m["max_rel"] <= MAX_REL and m["mean_abs"] <= MEAN_ABS, m
