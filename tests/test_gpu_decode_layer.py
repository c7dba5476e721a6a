"""Single-launch decode layer (K4f, pdscope_decode_layer) through the C-ABI.

The fused kernel keeps the per-lane arithmetic order of the three-launch
path (pdscope_route_topk + pdscope_swiglu_decode), so logits, ids, weights
and the layer output must be bitwise equal to it; the three-launch path is
itself checked against the oracle in test_gpu_kernels.py, and the fused
path is checked against the oracle here too (routing bit-exact given the
logits, output within bf16 tolerance).  The sync workspace must come back
zero with no wait having given up, also across hipGraph replays.
"""
import numpy as np
import pytest
import torch

from tests.gpu_helpers import (MAX_REL, MEAN_ABS, err_metrics, logits_within_accumulation_error,
                               oracle_layer_given_routing, u16)

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module")
def pd():
    from pdscope_amd import layer, ops, synthetic
    return ops, layer, synthetic


def _three_launch(ops, x, gate, slots, I, k, normalize, bias=None, merge="fused"):
    E, H = gate.shape
    logits = torch.empty((1, E), dtype=torch.bfloat16, device=DEV)
    ids = torch.empty((1, k), dtype=torch.int32, device=DEV)
    w = torch.empty((1, k), dtype=torch.bfloat16, device=DEV)
    ops.route_topk(x, gate, k, normalize, bias=bias, out=(logits, ids, w))
    h = torch.empty(k * I, dtype=torch.bfloat16, device=DEV)
    out = torch.empty((1, H), dtype=torch.bfloat16, device=DEV)
    ops.swiglu_decode(x, ids, w, slots, H, I, h, out, merge=merge)
    return logits, ids, w, out


def _fused(ops, x, gate, slots, I, k, normalize, bias=None, merge="fused"):
    E, H = gate.shape
    logits = torch.empty((1, E), dtype=torch.bfloat16, device=DEV)
    ids = torch.empty((1, k), dtype=torch.int32, device=DEV)
    w = torch.empty((1, k), dtype=torch.bfloat16, device=DEV)
    h = torch.empty(k * I, dtype=torch.bfloat16, device=DEV)
    out = torch.empty((1, H), dtype=torch.bfloat16, device=DEV)
    probs = torch.empty((1, E), dtype=torch.float32, device=DEV)
    ops.decode_layer(x, gate, slots, I, k, normalize, bias=bias, out=out, logits=logits, ids=ids, weights=w,
                     h_ws=h, probs=probs, merge=merge)
    return logits, ids, w, out, probs


def _assert_sync_clean(ops, H=2048):
    """No bounded wait gave up, and every block of the grid ran every launch
    (all per-block epochs equal)."""
    ws = ops.decode_workspace(DEV, H)
    torch.cuda.synchronize()
    words = ws.cpu().numpy()
    assert words[ops.DECODE_WS_ERROR_WORD] == 0, "a bounded wait of the fused decode kernel gave up"
    ep = words[:H // 4]
    assert ep[0] != 0 and (ep == ep[0]).all(), "per-block epochs diverged"


SHAPES = [
    dict(H=2048, I=768, E=128, k=8, normalize=True),    # Qwen3-30B-A3B
    dict(H=1024, I=512, E=64, k=4, normalize=True),
    dict(H=2048, I=1408, E=64, k=2, normalize=False),  # DeepSeek-V2-Lite widths, k within the fused limits
    dict(H=2048, I=512, E=256, k=8, normalize=True),   # 256 experts: four candidates per lane in the top-k
]


@pytest.mark.parametrize("merge", ["fused", "reference"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"H{s['H']}_I{s['I']}_E{s['E']}_k{s['k']}")
def test_fused_equals_three_launch(pd, shape, merge):
    ops, layer, synthetic = pd
    H, I, E, k, nrm = shape["H"], shape["I"], shape["E"], shape["k"], shape["normalize"]
    assert ops.decode_layer_supported(H, I, E, k, DEV), "the fused kernel should cover this shape"
    lay = synthetic.make_layer(H, I, E, k, nrm, seed=900 + H + I, device=DEV)
    slots = ops.slot_table([lay.experts[e] for e in range(E)], DEV)
    for seed in (1, 2, 3, 4):
        x = synthetic.make_tokens(1, H, seed=seed * 31 + E, device=DEV)
        a = _three_launch(ops, x, lay.gate, slots, I, k, nrm, merge=merge)
        b = _fused(ops, x, lay.gate, slots, I, k, nrm, merge=merge)
        torch.cuda.synchronize()
        for name, u, v in zip(("logits", "ids", "weights", "out"), a, b[:4]):
            assert torch.equal(u.view(torch.int16) if u.dtype == torch.bfloat16 else u,
                               v.view(torch.int16) if v.dtype == torch.bfloat16 else v), (name, seed)
    _assert_sync_clean(ops, H)


def test_fused_matches_oracle_qwen(orc, pd):
    ops, layer, synthetic = pd
    lay = synthetic.make_layer(**synthetic.QWEN, device=DEV)
    if not ops.decode_layer_supported(2048, 768, 128, 8, DEV):
        pytest.skip("shape not resident on this device")
    slots = ops.slot_table([lay.experts[e] for e in range(128)], DEV)
    experts = u16(lay.experts)
    for seed in (11, 12, 13):
        x = synthetic.make_tokens(1, 2048, seed=seed, device=DEV)
        logits, ids, w, out, probs = _fused(ops, x, lay.gate, slots, 768, 8, True)
        torch.cuda.synchronize()
        oi, ow, op = orc.route_from_logits(u16(logits), 8, True, None, want_probs=True)
        assert np.array_equal(ids.cpu().numpy(), oi)
        assert np.array_equal(u16(w), ow)
        assert np.array_equal(probs.cpu().numpy().view(np.uint32), op.view(np.uint32))
        exact = orc.route_logits(u16(x), u16(lay.gate))
        ok, _ = logits_within_accumulation_error(u16(logits), exact, u16(x), u16(lay.gate), orc.bf16_to_f32)
        assert ok, "logit mismatch beyond fp32 accumulation error"
        ref, _, _ = oracle_layer_given_routing(orc, u16(x), oi, ow, experts, 2048, 768)
        m = err_metrics(orc.bf16_to_f32(u16(out)), orc.bf16_to_f32(ref))
        assert m["max_rel"] <= MAX_REL and m["mean_abs"] <= MEAN_ABS, m
    _assert_sync_clean(ops)


COLLIDE_SHAPES = [dict(H=2048, I=768, E=128, k=8, big=[101, 7, 64]),
                  dict(H=2048, I=512, E=256, k=8, big=[200, 3, 129]),
                  dict(H=1024, I=512, E=64, k=4, big=[40, 9])]


@pytest.mark.parametrize("merge", ["fused", "reference"])
@pytest.mark.parametrize("shape", COLLIDE_SHAPES, ids=lambda s: f"E{s['E']}_k{s['k']}")
def test_fused_routing_where_logit_order_and_probability_order_differ(orc, pd, merge, shape):
    """The fused kernel picks experts by their bf16 logits first and checks
    the pick against the probabilities.  Here two or three experts get
    logits near +5 and the others distinct logits far below (their
    probabilities underflow to 0 and tie), so the probability top-k fills
    the rest with the lowest ids among the tied experts while the logit order
    would take the largest logits: the check must fail and the exact routing
    (and the rows it changes) must win.  Shapes cover 64, 128 and 256
    experts (the pick's two- and four-candidates-per-lane forms).  Ids and weights against
    the oracle, everything bitwise against the three-launch path."""
    ops, layer, synthetic = pd
    H, I, E, k, big = shape["H"], shape["I"], shape["E"], shape["k"], shape["big"]
    assert ops.decode_layer_supported(H, I, E, k, DEV), "the fused kernel should cover this shape"
    lay = synthetic.make_layer(H, I, E, k, True, seed=4242 + E, device=DEV)
    slots = ops.slot_table([lay.experts[e] for e in range(E)], DEV)
    x = synthetic.make_tokens(1, H, seed=77, device=DEV)
    xf = x.float()[0]
    target = torch.tensor([-130.0 - (e * 37) % 97 for e in range(E)])
    target[big] = torch.tensor([5.0, 4.5, 4.0][:len(big)])
    gate = (target[:, None].to(DEV) * xf[None, :] / (xf @ xf)).to(torch.bfloat16).contiguous()
    a = _three_launch(ops, x, gate, slots, I, k, True, merge=merge)
    b = _fused(ops, x, gate, slots, I, k, True, merge=merge)
    torch.cuda.synchronize()
    for name, u, v in zip(("logits", "ids", "weights", "out"), a, b[:4]):
        assert torch.equal(u.view(torch.int16) if u.dtype == torch.bfloat16 else u,
                           v.view(torch.int16) if v.dtype == torch.bfloat16 else v), name
    oi, ow = orc.route_from_logits(u16(b[0]), k, True, None)
    assert np.array_equal(b[1].cpu().numpy(), oi) and np.array_equal(u16(b[2]), ow)
    ids = b[1].cpu().numpy()[0].tolist()
    assert ids[:len(big)] == big
    assert ids[len(big):] == [e for e in range(E) if e not in big][:k - len(big)], ids
    lg = u16(b[0])[0].astype(np.int32)
    assert len(set(lg[[e for e in range(E) if e not in big]].tolist())) > 5, "the tied experts' logits must differ"
    _assert_sync_clean(ops, H)


def test_fused_zipf_bias_and_missing_copies(pd):
    """Router bias (Zipf workload) and slots without a ready copy (address 0 ->
    the expert contributes nothing) behave as on the three-launch path."""
    ops, layer, synthetic = pd
    lay = synthetic.make_layer(**synthetic.QWEN, seed=77, device=DEV)
    if not ops.decode_layer_supported(2048, 768, 128, 8, DEV):
        pytest.skip("shape not resident on this device")
    bias, _ = synthetic.zipf_bias(128, device=DEV)
    ptrs = [lay.experts[e].data_ptr() for e in range(128)]
    for e in range(0, 128, 3):
        ptrs[e] = 0
    slots = torch.tensor(ptrs, dtype=torch.int64, device=DEV)
    for seed in (5, 6, 7):
        x = synthetic.make_tokens(1, 2048, seed=seed, device=DEV)
        a = _three_launch(ops, x, lay.gate, slots, 768, 8, True, bias=bias)
        b = _fused(ops, x, lay.gate, slots, 768, 8, True, bias=bias)
        torch.cuda.synchronize()
        assert torch.equal(a[1], b[1])
        assert torch.equal(a[3].view(torch.int16), b[3].view(torch.int16))
    _assert_sync_clean(ops)


def test_fused_graph_replay(pd):
    """Captured once, replayed with new inputs: every replay equals eager, and
    the self-resetting counters leave the workspace clean."""
    ops, layer, synthetic = pd
    lay = synthetic.make_layer(**synthetic.QWEN, seed=78, device=DEV)
    if not ops.decode_layer_supported(2048, 768, 128, 8, DEV):
        pytest.skip("shape not resident on this device")
    slots = ops.slot_table([lay.experts[e] for e in range(128)], DEV)
    ws = layer.MoEWorkspace(1, 2048, 768, 128, 8, DEV)
    xin = synthetic.make_tokens(1, 2048, seed=100, device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        layer.moe_forward(xin, lay.gate, slots, ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        layer.moe_forward(xin, lay.gate, slots, ws)
    torch.cuda.synchronize()
    for seed in range(101, 109):
        x = synthetic.make_tokens(1, 2048, seed=seed, device=DEV)
        eager = _three_launch(ops, x, lay.gate, slots, 768, 8, True)
        torch.cuda.synchronize()
        xin.copy_(x)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(ws.ids[:1], eager[1])
        assert torch.equal(ws.out[:1].view(torch.int16), eager[3].view(torch.int16)), seed
    _assert_sync_clean(ops)


def test_decode_reference_merge_is_the_ordered_merge_of_the_expert_rows(orc, pd):
    """merge='reference' in both decode paths: the k expert outputs added in
    ascending expert id in bf16 arithmetic.  Each expert's output y_s is read
    off a k=1 decode call with weight 1.0 (bf16(1 * y_s) = y_s, and a slot's
    down dot product does not depend on k), and the layer output must equal
    the oracle's ordered merge of those rows bit for bit.  The grouped path's
    ordered merge is checked against the oracle on its own rows."""
    ops, layer, synthetic = pd
    H, I, E, k = 2048, 768, 128, 8
    lay = synthetic.make_layer(**synthetic.QWEN, seed=79, device=DEV)
    slots = ops.slot_table([lay.experts[e] for e in range(E)], DEV)
    one = torch.ones(1, dtype=torch.bfloat16, device=DEV)
    h = torch.empty(I, dtype=torch.bfloat16, device=DEV)
    ws = layer.MoEWorkspace(2, H, I, E, k, DEV)
    for seed in (21, 22, 23):
        x = synthetic.make_tokens(1, H, seed=seed, device=DEV)
        a = _three_launch(ops, x, lay.gate, slots, I, k, True, merge="reference")
        b = _fused(ops, x, lay.gate, slots, I, k, True, merge="reference")
        torch.cuda.synchronize()
        ids = a[1].cpu().numpy()[0]
        rank = np.argsort(np.argsort(ids)).astype(np.int32)   # grouped row of slot s: rank of its expert id
        y = np.empty((k, H), np.uint16)
        for s in range(k):
            ys = torch.empty((1, H), dtype=torch.bfloat16, device=DEV)
            ops.swiglu_decode(x, a[1][:, s:s + 1].contiguous(), one.view(1, 1), slots, H, I, h, ys)
            torch.cuda.synchronize()
            y[rank[s]] = u16(ys)[0]
        ref = orc.merge_ordered(y, rank, u16(a[2]))
        assert np.array_equal(u16(a[3]), ref), "three-launch decode, reference merge"
        assert np.array_equal(u16(b[3]), ref), "single-launch decode, reference merge"
        # grouped path, two tokens: ordered merge of its own expert rows
        x2 = torch.cat([x, synthetic.make_tokens(1, H, seed=seed + 50, device=DEV)])
        out2, _, ids2, w2 = layer.moe_forward(x2, lay.gate, slots, ws, merge="reference")
        torch.cuda.synchronize()
        p = orc.pack(ids2.cpu().numpy(), E)
        y2 = u16(ws.y[:2 * k * H]).reshape(2 * k, H)
        assert np.array_equal(u16(out2), orc.merge_ordered(y2, p["row_of"], u16(w2)))
    _assert_sync_clean(ops)


def test_unsupported_shape_falls_back(pd):
    """DeepSeek-V2-Lite top-6 with I=1408 exceeds the fused kernel's register
    plan: moe_forward falls back to route + decode GEMV, which still matches.
    So does H=4096 with three experts of 256, whose 1024 blocks cannot all be
    resident under the kernel's two-blocks-per-CU register budget."""
    ops, layer, synthetic = pd
    assert not ops.decode_layer_supported(4096, 256, 32, 3, DEV)
    lay = synthetic.make_layer(4096, 256, 32, 3, True, seed=6, device=DEV)
    slots = ops.slot_table([lay.experts[e] for e in range(32)], DEV)
    x = synthetic.make_tokens(1, 4096, seed=4, device=DEV)
    with pytest.raises(ValueError):
        _fused(ops, x, lay.gate, slots, 256, 3, True)
    ws = layer.MoEWorkspace(1, 4096, 256, 32, 3, DEV)
    out, _, ids, _ = layer.moe_forward(x, lay.gate, slots, ws)
    a = _three_launch(ops, x, lay.gate, slots, 256, 3, True)
    torch.cuda.synchronize()
    assert torch.equal(ids, a[1]) and torch.equal(out.view(torch.int16), a[3].view(torch.int16))
    assert not ops.decode_layer_supported(2048, 1408, 64, 6, DEV)
    lay = synthetic.make_layer(2048, 1408, 64, 6, False, seed=5, device=DEV)
    slots = ops.slot_table([lay.experts[e] for e in range(64)], DEV)
    x = synthetic.make_tokens(1, 2048, seed=3, device=DEV)
    with pytest.raises(ValueError):
        _fused(ops, x, lay.gate, slots, 1408, 6, False)
    ws = layer.MoEWorkspace(1, 2048, 1408, 64, 6, DEV)
    out, logits, ids, w = layer.moe_forward(x, lay.gate, slots, ws, normalize=False)
    a = _three_launch(ops, x, lay.gate, slots, 1408, 6, False)
    torch.cuda.synchronize()
    assert torch.equal(ids, a[1])
    assert torch.equal(out.view(torch.int16), a[3].view(torch.int16))


def _chained(ops, x, gate, slots, I, k, normalize, *, resid, next_gate, bias=None, merge="fused"):
    E, H = gate.shape
    r = dict(logits=torch.empty((1, E), dtype=torch.bfloat16, device=DEV),
             ids=torch.empty((1, k), dtype=torch.int32, device=DEV),
             weights=torch.empty((1, k), dtype=torch.bfloat16, device=DEV),
             h_ws=torch.empty(k * I, dtype=torch.bfloat16, device=DEV),
             out=torch.empty((1, H), dtype=torch.bfloat16, device=DEV),
             probs=torch.empty((1, E), dtype=torch.float32, device=DEV))
    extra = {}
    if resid is not None:
        extra.update(resid=resid, x_out=torch.empty((1, H), dtype=torch.bfloat16, device=DEV))
    if next_gate is not None:
        extra.update(next_gate=next_gate, pred_out=torch.full((k,), -7, dtype=torch.int32, device=DEV))
    ops.decode_layer(x, gate, slots, I, k, normalize, bias=bias, merge=merge, **r, **extra)
    r.update(extra)
    return r


def _route_ids(ops, x, gate, k, normalize):
    E = gate.shape[0]
    ids = torch.empty((1, k), dtype=torch.int32, device=DEV)
    ops.route_topk(x, gate, k, normalize, out=(torch.empty((1, E), dtype=torch.bfloat16, device=DEV), ids,
                                                torch.empty((1, k), dtype=torch.bfloat16, device=DEV)))
    return ids


CHAIN_SHAPES = [dict(H=2048, I=768, E=128, k=8, normalize=True),
                dict(H=1024, I=512, E=64, k=4, normalize=True),
                dict(H=2048, I=512, E=256, k=8, normalize=True)]


@pytest.mark.parametrize("merge", ["fused", "reference"])
@pytest.mark.parametrize("shape", CHAIN_SHAPES, ids=lambda s: f"H{s['H']}_E{s['E']}_k{s['k']}")
def test_chained_equals_plain_launch_on_the_residual_sum(pd, shape, merge):
    """pdscope_decode_layer_chained: every output is bitwise that of
    pdscope_decode_layer on x_eff = bf16(x + resid); x_out holds x_eff, and
    pred_out the ids pdscope_route_topk gives for the next gate on x_eff (no
    bias).  With only one of the two extras given the rest is unchanged."""
    ops, layer, synthetic = pd
    H, I, E, k, nrm = shape["H"], shape["I"], shape["E"], shape["k"], shape["normalize"]
    lay = synthetic.make_layer(H, I, E, k, nrm, seed=1200 + E, device=DEV)
    nxt = synthetic.make_layer(H, 8, E, k, nrm, seed=1300 + E, device=DEV).gate
    slots = ops.slot_table([lay.experts[e] for e in range(E)], DEV)
    for seed in (1, 2, 3):
        x = synthetic.make_tokens(1, H, seed=seed * 7 + E, device=DEV)
        resid = synthetic.make_tokens(1, H, seed=seed * 7 + E + 500, device=DEV)
        x_eff = x + resid                                   # fp32 sum, one bf16 rounding
        base = _fused(ops, x_eff, lay.gate, slots, I, k, nrm, merge=merge)
        h_base = torch.empty(k * I, dtype=torch.bfloat16, device=DEV)
        ops.decode_layer(x_eff, lay.gate, slots, I, k, nrm, out=torch.empty_like(base[3]),
                         logits=torch.empty_like(base[0]), ids=torch.empty_like(base[1]),
                         weights=torch.empty_like(base[2]), h_ws=h_base, merge=merge)
        nids = _route_ids(ops, x_eff, nxt, k, nrm)
        torch.cuda.synchronize()
        for kind, rs, ng in (("both", resid, nxt), ("resid", resid, None), ("predictor", None, nxt)):
            xin = x if rs is not None else x_eff
            c = _chained(ops, xin, lay.gate, slots, I, k, nrm, resid=rs, next_gate=ng, merge=merge)
            torch.cuda.synchronize()
            checks = [("logits", base[0]), ("ids", base[1]), ("weights", base[2]), ("out", base[3]),
                      ("probs", base[4]), ("h_ws", h_base)]
            if rs is not None:
                checks.append(("x_out", x_eff))
            for name, want in checks:
                got = c[name]
                eq = torch.equal(got.view(torch.int16), want.view(torch.int16)) if got.dtype == torch.bfloat16 \
                    else torch.equal(got.view(torch.int32), want.view(torch.int32))
                assert eq, (kind, name, seed)
            if ng is not None:
                assert torch.equal(c["pred_out"], nids[0]), (kind, seed)
    _assert_sync_clean(ops, H)


def _colliding_gate(x_eff, E, big, scores):
    """Router rows whose logits on x_eff are about `scores` for the experts in
    `big` and distinct values far below for the rest (probabilities 0)."""
    xf = x_eff.float()[0]
    target = torch.tensor([-130.0 - (e * 37) % 97 for e in range(E)])
    target[big] = torch.tensor(scores)
    return (target[:, None].to(DEV) * xf[None, :] / (xf @ xf)).to(torch.bfloat16).contiguous()


CHAIN_COLLIDE = [dict(H=2048, I=768, E=128, k=8, big=[30, 99, 2], nbig=[12, 127]),
                 dict(H=2048, I=512, E=256, k=8, big=[250, 1, 130], nbig=[200, 17])]


@pytest.mark.parametrize("merge", ["fused", "reference"])
@pytest.mark.parametrize("shape", CHAIN_COLLIDE, ids=lambda s: f"E{s['E']}")
def test_chained_routing_where_logit_order_and_probability_order_differ(pd, merge, shape):
    """The chained kernel on logits whose probabilities tie at 0 below the
    top three (the logit-key pick fails its check and the exact routing and
    its rows replace it), with the next gate built the same way: every output
    bitwise that of the plain launch on x_eff, pred_out the exact routing of
    the next gate."""
    ops, layer, synthetic = pd
    H, I, E, k, big, nbig = shape["H"], shape["I"], shape["E"], shape["k"], shape["big"], shape["nbig"]
    assert ops.decode_layer_supported(H, I, E, k, DEV), "the fused kernel should cover this shape"
    lay = synthetic.make_layer(H, I, E, k, True, seed=4343 + E, device=DEV)
    slots = ops.slot_table([lay.experts[e] for e in range(E)], DEV)
    x = synthetic.make_tokens(1, H, seed=78, device=DEV)
    resid = synthetic.make_tokens(1, H, seed=79, device=DEV)
    x_eff = x + resid
    gate = _colliding_gate(x_eff, E, big, [5.0, 4.5, 4.0])
    nxt = _colliding_gate(x_eff, E, nbig, [3.0, 2.5])
    base = _fused(ops, x_eff, gate, slots, I, k, True, merge=merge)
    nids = _route_ids(ops, x_eff, nxt, k, True)
    c = _chained(ops, x, gate, slots, I, k, True, resid=resid, next_gate=nxt, merge=merge)
    torch.cuda.synchronize()
    for name, want in (("logits", base[0]), ("ids", base[1]), ("weights", base[2]), ("out", base[3]),
                       ("probs", base[4]), ("x_out", x_eff)):
        got = c[name]
        eq = torch.equal(got.view(torch.int16), want.view(torch.int16)) if got.dtype == torch.bfloat16 \
            else torch.equal(got.view(torch.int32), want.view(torch.int32))
        assert eq, name
    ids = c["ids"].cpu().numpy()[0].tolist()
    assert ids == big + [e for e in range(E) if e not in big][:k - 3], ids
    assert torch.equal(c["pred_out"], nids[0])
    assert c["pred_out"].cpu().tolist() == nbig + [e for e in range(E) if e not in nbig][:k - 2]
    _assert_sync_clean(ops, H)


def test_chain_of_layers_equals_layer_by_layer(pd):
    """Four layers chained the way a decode step runs them: each launch takes
    the previous output and residual and predicts the next layer's experts.
    Equal to plain launches on the explicit residual sums; pred_out of each
    layer is the next gate's routing of that layer's input.  Launches
    without a next gate in between keep the predictor words current (the
    next predicting launch still waits for this launch's words)."""
    ops, layer, synthetic = pd
    H, I, E, k = 2048, 768, 128, 8
    layers = [synthetic.make_layer(**dict(synthetic.QWEN, seed=90 + l), device=DEV) for l in range(4)]
    slots = [ops.slot_table([ly.experts[e] for e in range(E)], DEV) for ly in layers]
    x0 = synthetic.make_tokens(1, H, seed=41, device=DEV)
    r0 = synthetic.make_tokens(1, H, seed=42, device=DEV)
    x, resid = x0, r0
    outs = []
    for l, ly in enumerate(layers):
        nxt = layers[l + 1].gate if l + 1 < len(layers) else None
        c = _chained(ops, x, ly.gate, slots[l], I, k, True, resid=resid, next_gate=nxt, merge="reference")
        outs.append(c)
        x, resid = c["out"], c["x_out"]
    torch.cuda.synchronize()
    x, resid = x0, r0
    for l, ly in enumerate(layers):
        x_eff = x + resid
        b = _fused(ops, x_eff, ly.gate, slots[l], I, k, True, merge="reference")
        torch.cuda.synchronize()
        assert torch.equal(outs[l]["x_out"].view(torch.int16), x_eff.view(torch.int16)), l
        assert torch.equal(outs[l]["ids"], b[1]), l
        assert torch.equal(outs[l]["out"].view(torch.int16), b[3].view(torch.int16)), l
        if l + 1 < len(layers):
            nids = _route_ids(ops, x_eff, layers[l + 1].gate, k, True)
            torch.cuda.synchronize()
            assert torch.equal(outs[l]["pred_out"], nids[0]), l
        x, resid = b[3], x_eff
    _assert_sync_clean(ops, H)


def test_chained_argument_checks(pd):
    ops, layer, synthetic = pd
    H, I, E, k = 2048, 768, 128, 8
    lay = synthetic.make_layer(**synthetic.QWEN, seed=82, device=DEV)
    slots = ops.slot_table([lay.experts[e] for e in range(E)], DEV)
    x = synthetic.make_tokens(1, H, seed=1, device=DEV)
    args = dict(out=torch.empty((1, H), dtype=torch.bfloat16, device=DEV),
                logits=torch.empty((1, E), dtype=torch.bfloat16, device=DEV),
                ids=torch.empty((1, k), dtype=torch.int32, device=DEV),
                weights=torch.empty((1, k), dtype=torch.bfloat16, device=DEV),
                h_ws=torch.empty(k * I, dtype=torch.bfloat16, device=DEV))
    with pytest.raises(ValueError):          # resid without x_out
        ops.decode_layer(x, lay.gate, slots, I, k, True, resid=x, **args)
    with pytest.raises(ValueError):          # pred_out without next_gate
        ops.decode_layer(x, lay.gate, slots, I, k, True, pred_out=args["ids"][0], **args)
    with pytest.raises(ValueError):          # next gate of another shape
        ops.decode_layer(x, lay.gate, slots, I, k, True, next_gate=lay.gate[:64].contiguous(),
                         pred_out=args["ids"][0].clone(), **args)
    with pytest.raises(ValueError):          # pred_out of the wrong length
        ops.decode_layer(x, lay.gate, slots, I, k, True, next_gate=lay.gate,
                         pred_out=args["ids"][0, :3].contiguous(), **args)
    # the predictor needs E <= H/2: 256 experts over H = 256 (64 blocks) is refused by the library
    small = synthetic.make_layer(256, 64, 256, 2, True, seed=3, device=DEV)
    sl = ops.slot_table([small.experts[e] for e in range(256)], DEV)
    xs = synthetic.make_tokens(1, 256, seed=2, device=DEV)
    with pytest.raises(ValueError):
        ops.decode_layer(xs, small.gate, sl, 64, 2, True, next_gate=small.gate,
                         pred_out=torch.empty(2, dtype=torch.int32, device=DEV),
                         out=torch.empty((1, 256), dtype=torch.bfloat16, device=DEV),
                         logits=torch.empty((1, 256), dtype=torch.bfloat16, device=DEV),
                         ids=torch.empty((1, 2), dtype=torch.int32, device=DEV),
                         weights=torch.empty((1, 2), dtype=torch.bfloat16, device=DEV),
                         h_ws=torch.empty(128, dtype=torch.bfloat16, device=DEV))


def test_chained_graph_replay(pd):
    """A four-layer chained step captured once and replayed with new inputs:
    every replay equals the eager chain (outputs, residuals, predictions), with
    eager work and synchronisations between the replays, and the workspace
    stays clean."""
    ops, layer, synthetic = pd
    H, I, E, k = 2048, 768, 128, 8
    layers = [synthetic.make_layer(**dict(synthetic.QWEN, seed=70 + l), device=DEV) for l in range(4)]
    slots = [ops.slot_table([ly.experts[e] for e in range(E)], DEV) for ly in layers]
    xin = synthetic.make_tokens(1, H, seed=300, device=DEV)
    rin = synthetic.make_tokens(1, H, seed=301, device=DEV)
    bufs = [dict(out=torch.empty((1, H), dtype=torch.bfloat16, device=DEV),
                 x_out=torch.empty((1, H), dtype=torch.bfloat16, device=DEV),
                 logits=torch.empty((1, E), dtype=torch.bfloat16, device=DEV),
                 ids=torch.empty((1, k), dtype=torch.int32, device=DEV),
                 weights=torch.empty((1, k), dtype=torch.bfloat16, device=DEV),
                 h_ws=torch.empty(k * I, dtype=torch.bfloat16, device=DEV),
                 pred=torch.full((k,), -1, dtype=torch.int32, device=DEV)) for _ in layers]

    def step():
        x, r = xin, rin
        for l, ly in enumerate(layers):
            b = bufs[l]
            extra = dict(next_gate=layers[l + 1].gate, pred_out=b["pred"]) if l + 1 < len(layers) else {}
            ops.decode_layer(x, ly.gate, slots[l], I, k, True, out=b["out"], logits=b["logits"], ids=b["ids"],
                             weights=b["weights"], h_ws=b["h_ws"], resid=r, x_out=b["x_out"], merge="reference",
                             **extra)
            x, r = b["out"], b["x_out"]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()
    for seed in range(310, 316):
        xin.copy_(synthetic.make_tokens(1, H, seed=seed, device=DEV))
        rin.copy_(synthetic.make_tokens(1, H, seed=seed + 100, device=DEV))
        step()
        torch.cuda.synchronize()
        eager = [{n: t.clone() for n, t in b.items() if n != "h_ws"} for b in bufs]
        for b in bufs:
            for t in b.values():
                t.zero_()
        g.replay()
        torch.cuda.synchronize()
        for l, (b, e) in enumerate(zip(bufs, eager)):
            for n, want in e.items():
                if n == "pred" and l + 1 == len(layers):
                    continue
                assert torch.equal(b[n], want), (seed, l, n)
    _assert_sync_clean(ops, H)


def test_bound_decode_equals_the_chained_launch_and_reads_back(pd):
    """ops.DecodeBinding (pdscope_decode_bind / _run): each token's out,
    logits, weights and int64 ids equal pdscope_decode_layer_chained with the
    same arguments bit for bit; the read-back words in pinned host memory
    hold the routed ids, the next-layer prediction and a clear error word,
    each tagged with the call's number, for several tokens in a row; a
    binding without a next gate leaves the prediction words alone.  Bad host
    buffers and numbers are rejected."""
    import ctypes

    from pdscope_amd import _lib
    ops, layer, synthetic = pd
    H, I, E, k = 2048, 768, 128, 8
    l0 = synthetic.make_layer(**dict(synthetic.QWEN, seed=80), device=DEV)
    l1 = synthetic.make_layer(**dict(synthetic.QWEN, seed=81), device=DEV)
    slots = ops.slot_table([l0.experts[e] for e in range(E)], DEV)
    host = torch.full((64,), -7, dtype=torch.int32, pin_memory=True)
    bound = ops.DecodeBinding(l0.gate, slots, I, k, True, host=host, error_at=40, merge="reference",
                              next_gate=l1.gate)
    plain = ops.DecodeBinding(l0.gate, slots, I, k, True, host=host, ids_at=20, error_at=41, merge="reference")
    try:
        for seed in range(400, 404):
            x = synthetic.make_tokens(1, H, seed=seed, device=DEV)
            got = dict(out=torch.empty((1, H), dtype=torch.bfloat16, device=DEV),
                       logits=torch.empty((1, E), dtype=torch.bfloat16, device=DEV),
                       weights=torch.empty((1, k), dtype=torch.bfloat16, device=DEV),
                       selected=torch.empty((1, k), dtype=torch.int64, device=DEV))
            tag = seed - 399
            bound.run(x, got["out"], got["logits"], got["weights"], got["selected"], seq=tag)
            pout = torch.empty((1, H), dtype=torch.bfloat16, device=DEV)
            plain.run(x, pout, torch.empty((1, E), dtype=torch.bfloat16, device=DEV),
                      torch.empty((1, k), dtype=torch.bfloat16, device=DEV), seq=tag + 1000)
            want = dict(out=torch.empty((1, H), dtype=torch.bfloat16, device=DEV),
                        logits=torch.empty((1, E), dtype=torch.bfloat16, device=DEV),
                        ids=torch.empty((1, k), dtype=torch.int32, device=DEV),
                        weights=torch.empty((1, k), dtype=torch.bfloat16, device=DEV),
                        pred=torch.empty((k,), dtype=torch.int32, device=DEV))
            ops.decode_layer(x, l0.gate, slots, I, k, True, out=want["out"], logits=want["logits"],
                             ids=want["ids"], weights=want["weights"],
                             h_ws=torch.empty(k * I, dtype=torch.bfloat16, device=DEV), merge="reference",
                             next_gate=l1.gate, pred_out=want["pred"])
            torch.cuda.synchronize()
            for n in ("out", "logits", "weights"):
                assert torch.equal(got[n], want[n]), (seed, n)
            assert torch.equal(pout, want["out"]), seed
            assert torch.equal(got["selected"], want["ids"].long()), seed
            words = host.numpy().tolist()
            untag = ops.DecodeBinding.tagged_words
            assert untag(words[:k], tag) == want["ids"][0].tolist(), seed
            assert untag(words[k:2 * k], tag) == want["pred"].tolist(), seed
            assert untag(words[20:20 + k], tag + 1000) == want["ids"][0].tolist(), seed
            assert words[20 + k:20 + 2 * k] == [-7] * k, seed   # no next gate bound
            assert untag(words[40:41], tag) == [0] and untag(words[41:42], tag + 1000) == [0], seed
        for bad in (0, 0x8000):   # a number outside 1 .. 32767 is refused before any launch
            with pytest.raises(ValueError, match="seq must be"):
                plain.run(x, pout, got["logits"], got["weights"], seq=bad)
    finally:
        bound.close()
        plain.close()
    with pytest.raises(ValueError, match="closed"):
        bound.run(x, got["out"], got["logits"], got["weights"])
    with pytest.raises(ValueError, match="pinned"):
        ops.DecodeBinding(l0.gate, slots, I, k, True, host=torch.zeros(64, dtype=torch.int32), error_at=40)
    with pytest.raises(ValueError, match="overlapping"):
        ops.DecodeBinding(l0.gate, slots, I, k, True, host=host, error_at=3)

    # the C-ABI itself refuses read-back words outside pinned host memory
    plain_words = (ctypes.c_int32 * 32)()
    handle = ctypes.c_void_p()
    h_ws = torch.empty(k * I, dtype=torch.bfloat16, device=DEV)
    ids = torch.empty(k, dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError, match="pinned host memory"):
        _lib.call("pdscope_decode_bind", l0.gate.data_ptr(), None, H, E, k, 1, 1, slots.data_ptr(), I, None, None,
                  ids.data_ptr(), None, h_ws.data_ptr(), ops.decode_workspace(DEV, H).data_ptr(),
                  ctypes.addressof(plain_words), ctypes.addressof(plain_words) + 64, ctypes.byref(handle))
    assert handle.value is None
    _assert_sync_clean(ops, H)
