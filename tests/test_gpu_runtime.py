"""GPU tests of the drop-in runtime (PDScopeCudaRuntime), executor staging and native dispatch.

Every layer output is compared with the oracle applied to the runtime's own
routing (ids/weights, themselves checked bit-exact against the oracle on
the returned logits).  Ledger closure (transfers completed, no demand left
open, every routed expert completed once) is asserted after each sequence.
"""
import ctypes

import numpy as np
import pytest
import torch

from tests.gpu_helpers import assert_layer_close, oracle_layer_given_routing, u16

pytestmark = pytest.mark.gpu
DEV = "cuda"


def build(n_layers, H, I, E, k, seed=77):
    from pdscope_amd import synthetic
    from pdscope_amd.executor import masters_from_block
    layers = [synthetic.make_layer(H, I, E, k, True, seed=seed + 100 * l, device=DEV) for l in range(n_layers)]
    masters = {}
    for l, lay in enumerate(layers):
        masters.update(masters_from_block(l, lay.experts, E, H, I))
    return layers, masters


def check_output(orc, out, routing, x, layer_obj, H, I, k, normalize=True, row=None, merge=None):
    """Routing bit-exact against the oracle given the logits, and the output
    within tolerance of the oracle layer with the runtime's merge (taken from
    the trace row when `merge` is not given)."""
    if merge is None and row is not None:
        merge = row["merge_mode"]
    if merge is None:
        raise ValueError("check_output needs the runtime's merge mode (merge= or row=)")
    ids = routing.selected.cpu().numpy()
    oi, ow = orc.route_from_logits(u16(routing.logits), k, normalize)
    assert np.array_equal(ids, oi) and np.array_equal(u16(routing.weights), ow)
    ref, _, _ = oracle_layer_given_routing(orc, u16(x), ids, u16(routing.weights), u16(layer_obj.experts), H, I,
                                           merge=merge)
    try:
        assert_layer_close(orc, out, ref)
    except AssertionError as err:
        # name the experts behind the mismatch: those routed by every badly
        # matching token, with where the runtime placed them
        d = np.abs(orc.bf16_to_f32(u16(out)).astype(np.float64) - orc.bf16_to_f32(ref))
        bad = np.nonzero(d.max(axis=1) > 0.1 * np.abs(orc.bf16_to_f32(ref)).max())[0]
        common = set(ids[bad[0]]) if len(bad) else set()
        for t in bad[1:]:
            common &= set(ids[t])
        # experts every one of whose tokens is off (the likely culprits)
        badset = set(bad.tolist())
        suspects = sorted(e for e in set(ids.reshape(-1).tolist())
                          if all(t in badset for t in np.nonzero((ids == e).any(axis=1))[0]))
        where = {}
        if row is not None:
            dec = row["decision"]
            demand = list(dec["on_demand_queue"])

            def place(e):
                if e in dec["gpu_resident_queue"]:
                    return "resident"
                return f"staged#{demand.index(e)}" if e in demand else "cpu"
            where = {e: place(e) for e in sorted(common | set(suspects))}
        raise AssertionError(f"{err}; {len(bad)} of {ids.shape[0]} tokens off, experts common to all of them: "
                             f"{sorted(common)}, experts with all their tokens off: {suspects}; placement {where}"
                             ) from None


def watch_copies(rt, layers):
    """Compare every device copy with its layer's weights on the compute
    stream right before the launch that reads it (no host sync); returns the
    list of (key, mismatch flag tensor) to check after synchronising."""
    records = []

    def hook(key, flat):
        w = layers[key.layer].experts[key.expert]
        got = flat[:w.numel() * 2].view(torch.int16)
        records.append((key, (got != w.view(torch.int16)).any()))
    rt.executor.consume_hook = hook
    return records


def assert_copies_intact(records):
    bad = [(k.layer, k.expert) for k, m in records if bool(m)]
    records.clear()
    assert not bad, f"device copies differ from their masters when consumed: {bad}"


def explain_rows(orc, rt, x, layer_obj, layer, ids, H, I, k):
    """After a mismatch: which experts' grouped output rows (ws.y) differ
    from the oracle's expert outputs, whether the device grouping equals the
    oracle's, and the device/host slot-table entries of those experts."""
    ws = rt._ws[k]
    T = x.shape[0]
    p = orc.pack(np.ascontiguousarray(ids, dtype=np.int32), layer_obj.E)
    offs = ws.offsets.cpu().numpy()
    perm = ws.perm_token[:T * k].cpu().numpy()
    same_pack = bool(np.array_equal(offs, p["offsets"]) and np.array_equal(perm, p["perm_token"]))
    y = u16(ws.y[:T * k * H].view(T * k, H))
    xg = u16(x)[p["perm_token"]]
    experts = u16(layer_obj.experts)
    IH = I * H
    wrong = []
    for e in np.nonzero(p["counts"])[0]:
        a, b = p["offsets"][e], p["offsets"][e + 1]
        blk = experts[e]
        ref = orc.expert_forward(xg[a:b], blk[:IH].reshape(I, H), blk[IH:2 * IH].reshape(I, H),
                                 blk[2 * IH:].reshape(H, I))
        d = np.abs(orc.bf16_to_f32(y[a:b]).astype(np.float64) - orc.bf16_to_f32(ref))
        if d.max() > 0.1 * np.abs(orc.bf16_to_f32(ref)).max():
            wrong.append(int(e))
    dev_tab, host_tab = rt.executor.table(layer, layer_obj.E)
    dev_tab = dev_tab.cpu().tolist()
    tabs = {e: (hex(dev_tab[e]), hex(host_tab[e])) for e in wrong[:6]}
    return f"grouping equals the oracle's: {same_pack}; experts with wrong y rows: {wrong}; tables {tabs}"


def closure(rt):
    st = rt.cache.stats()
    assert st.get("h2d_bytes_submitted", 0) == st.get("h2d_bytes_completed", 0)
    assert rt.cache.active_demand is None
    assert not rt.executor.loads and not rt.executor.computes


def test_runtime_prefill_then_decode_with_staging_and_prefetch(orc):
    from pdscope_amd import synthetic
    from pdscope_amd.cache import ExpertKey
    from pdscope_amd.pdscope_runtime import PDScopeCudaRuntime
    H, I, E, k = 256, 128, 32, 4
    layers, masters = build(2, H, I, E, k)
    hot = [ExpertKey(l, e, "bf16") for l in range(2) for e in range(6)]
    rt = PDScopeCudaRuntime(masters, hot_keys=hot, speculative_slots=4, demand_slots=2)
    gen = torch.Generator(device=DEV).manual_seed(3)
    try:
        for step, T in enumerate((16, 1, 1, 1)):
            x = (torch.randn((T, H), generator=gen, device=DEV)).to(torch.bfloat16)
            for l in range(2):
                out, routing, row = rt.forward(x, layers[l].gate, layer=l, step=step, next_gate=
                                               layers[l + 1].gate if l + 1 < 2 else None, top_k=k)
                torch.cuda.synchronize()
                check_output(orc, out, routing, x, layers[l], H, I, k, merge=rt.merge)
                assert set(row["decision"]["gpu_resident_queue"]) | set(row["decision"]["on_demand_queue"]) == \
                    set(row["token_counts"])
                x = torch.nn.functional.layer_norm((out.float() + x.float()), (H,)).to(torch.bfloat16)
        closure(rt)
        st = rt.cache.stats()
        assert st.get("demand_loads_submitted", 0) > 0          # misses went through staging
        assert st.get("prefetch_loads_submitted", 0) > 0        # the predictor prefetched
        assert all(rt.cache.lookup(h) is not None for h in hot)  # hot set intact
    finally:
        rt.close()


def test_runtime_qwen_demand_staging_eight_slots(orc):
    from pdscope_amd import synthetic
    from pdscope_amd.cache import ExpertKey
    from pdscope_amd.pdscope_runtime import PDScopeCudaRuntime
    q = synthetic.QWEN
    layers, masters = build(1, q["H"], q["I"], q["E"], q["k"], seed=91)
    hot = [ExpertKey(0, e, "bf16") for e in range(32)]
    rt = PDScopeCudaRuntime(masters, hot_keys=hot, speculative_slots=0, demand_slots=8)
    copies = watch_copies(rt, layers)
    try:
        x = synthetic.make_tokens(64, q["H"], seed=92)
        out, routing, row = rt.forward(x, layers[0].gate, layer=0, step=0, top_k=8)
        torch.cuda.synchronize()
        assert_copies_intact(copies)
        check_output(orc, out, routing, x, layers[0], q["H"], q["I"], 8, row=row)
        assert len(row["decision"]["on_demand_queue"]) > 50
        assert {p["slot"] for p in row["ping_pong_slots"]} <= set(range(8))
        closure(rt)
    finally:
        rt.close()


def test_runtime_staging_slots_reused_across_calls(orc):
    """Successive prefill calls stage different experts through the same eight
    slots (each slot's previous contents were other weights, read by earlier
    launches): every call matches the oracle."""
    from pdscope_amd import synthetic
    from pdscope_amd.cache import ExpertKey
    from pdscope_amd.pdscope_runtime import PDScopeCudaRuntime
    q = synthetic.QWEN
    layers, masters = build(2, q["H"], q["I"], q["E"], q["k"], seed=95)
    hot = [ExpertKey(l, e, "bf16") for l in range(2) for e in range(16)]
    rt = PDScopeCudaRuntime(masters, hot_keys=hot, speculative_slots=0, demand_slots=8)
    copies = watch_copies(rt, layers)
    try:
        for call in range(4):
            l = call % 2
            x = synthetic.make_tokens(48 + 16 * call, q["H"], seed=96 + call)
            out, routing, row = rt.forward(x, layers[l].gate, layer=l, step=0, top_k=8, request=f"r{call}")
            torch.cuda.synchronize()
            assert_copies_intact(copies)
            try:
                check_output(orc, out, routing, x, layers[l], q["H"], q["I"], 8, row=row)
            except AssertionError as err:
                why = explain_rows(orc, rt, x, layers[l], l, routing.selected.cpu().numpy(), q["H"], q["I"], 8)
                raise AssertionError(f"call {call}: {err}; {why}") from None
            assert len(row["decision"]["on_demand_queue"]) > 40
        closure(rt)
    finally:
        rt.close()


@pytest.mark.parametrize("case", ["zipf_staged", "uniform_resident"])
def test_runtime_t4096_sampled_tokens(orc, case):
    """T=4096 prefill layers through the runtime at full size.  zipf_staged:
    a Zipf(1.1) router bias, the 32 hottest experts resident, every other
    touched expert staged through 8 demand slots in batches, hot experts
    spanning many row tiles.  uniform_resident: uniform routing with all 128
    experts resident, one grouped launch on 384-row gate/up tiles and
    256-row down tiles.  Routing is checked bit-exact for every token; for a
    seeded sample of tokens each of their grouped rows is checked against the
    oracle's expert output and their merged outputs against the oracle merge
    of those rows."""
    from pdscope_amd import synthetic
    from pdscope_amd.cache import ExpertKey
    from pdscope_amd.pdscope_runtime import PDScopeCudaRuntime
    from tests.gpu_helpers import MAX_REL, MEAN_ABS, err_metrics
    q = synthetic.QWEN
    H, I, E, k, T = q["H"], q["I"], q["E"], q["k"], 4096
    layers, masters = build(1, H, I, E, k, seed=97)
    zipf = case == "zipf_staged"
    bias, perm = synthetic.zipf_bias(E, 1.1, seed=98, device=DEV)
    hottest = sorted(range(E), key=lambda e: int(perm[e]))[:32] if zipf else list(range(E))
    if not zipf:
        bias = None
    rt = PDScopeCudaRuntime(masters, hot_keys=[ExpertKey(0, e, "bf16") for e in hottest], speculative_slots=0,
                            demand_slots=8)
    copies = watch_copies(rt, layers)
    try:
        x = synthetic.make_tokens(T, H, seed=99)
        out, routing, row = rt.forward(x, layers[0].gate, layer=0, step=0, top_k=k, bias=bias)
        torch.cuda.synchronize()
        assert_copies_intact(copies)
        ids, wk = routing.selected.cpu().numpy(), u16(routing.weights)
        oi, ow = orc.route_from_logits(u16(routing.logits), k, True, None if bias is None else bias.cpu().numpy())
        assert np.array_equal(ids, oi) and np.array_equal(wk, ow)
        counts = np.bincount(ids.reshape(-1), minlength=E)
        if zipf:
            assert counts.max() > 2000 and len(row["decision"]["on_demand_queue"]) > 50
        else:
            from pdscope_amd import layer as L, ops
            assert not row["decision"]["on_demand_queue"]
            bm = ops.grouped_block_m(T * k // E, int(counts.max()))
            assert bm == 384 and L.down_block_m(bm, H, I) == 256
        ws = rt._ws[k]
        row_of = ws.row_of[:T * k].cpu().numpy().reshape(T, k)
        y_all = u16(ws.y[:T * k * H].view(T * k, H))
        rng = np.random.default_rng(4097)
        tokens = np.sort(rng.choice(T, 32, replace=False))
        experts, xu, IH = u16(layers[0].experts), u16(x), I * H
        got_y, ref_y = [], []
        for t in tokens:
            for s in range(k):
                blk = experts[ids[t, s]]
                ref_y.append(orc.expert_forward(xu[t:t + 1], blk[:IH].reshape(I, H), blk[IH:2 * IH].reshape(I, H),
                                                blk[2 * IH:].reshape(H, I))[0])
                got_y.append(y_all[row_of[t, s]])
        got_y, ref_y = np.stack(got_y), np.stack(ref_y)
        m_y = err_metrics(orc.bf16_to_f32(got_y), orc.bf16_to_f32(ref_y))
        assert m_y["max_rel"] <= MAX_REL and m_y["mean_abs"] <= MEAN_ABS, m_y
        # the runtime's default merge (merge='reference'): each sampled token's
        # device rows added in ascending expert id in bf16, bit for bit
        assert rt.merge == "reference"
        rank = np.argsort(np.argsort(row_of[tokens], axis=1), axis=1)      # order of a token's grouped rows
        local = (np.arange(len(tokens))[:, None] * k + rank).astype(np.int32)
        y_local = np.empty_like(got_y)
        y_local[local.reshape(-1)] = got_y
        assert np.array_equal(u16(out)[tokens], orc.merge_ordered(y_local, local, wk[tokens]))
        closure(rt)
    finally:
        rt.close()


def test_slot_table_fill_is_ordered_before_uploads_on_other_streams():
    """The device slot table is created by a zero fill on the caller's
    stream; its first upload runs on the compute stream.  With the caller's
    stream busy (a timed spin kernel ahead of the fill), the upload must
    still be what the table holds afterwards."""
    from pdscope_amd.cache import ExpertKey
    from pdscope_amd.pdscope_runtime import PDScopeCudaRuntime
    H, I, E, k = 256, 128, 32, 4
    layers, masters = build(2, H, I, E, k, seed=81)
    rt = PDScopeCudaRuntime(masters, hot_keys=[ExpertKey(1, e, "bf16") for e in range(4)], speculative_slots=0)
    try:
        ex = rt.executor
        torch.cuda.synchronize()
        assert 1 not in ex._dev_tables
        torch.cuda._sleep(20_000_000)  # about 10 ms on the caller's stream
        dev = ex.upload_table(1, E, ex.compute_stream)
        ex.compute_stream.synchronize()
        torch.cuda.synchronize()
        host = ex.table(1, E)[1]
        assert all(host[e] != 0 for e in range(4))
        assert dev.cpu().tolist() == list(host)
    finally:
        rt.close()


def test_runtime_bound_decode_matches_the_single_launch_layer(orc):
    """resident_graphs=True serves decode tokens through the layer's bound
    launch: output and routing equal the single-launch layer bit for bit, and
    each call returns routing tensors of its own (later calls leave them as
    they were)."""
    from pdscope_amd import layer, ops, synthetic
    from pdscope_amd.cache import ExpertKey
    from pdscope_amd.pdscope_runtime import PDScopeCudaRuntime
    q = synthetic.QWEN
    layers, masters = build(1, q["H"], q["I"], q["E"], q["k"], seed=93)
    hot = [ExpertKey(0, e, "bf16") for e in range(q["E"])]
    rt = PDScopeCudaRuntime(masters, hot_keys=hot, speculative_slots=0, resident_graphs=True)
    slots = ops.slot_table([layers[0].experts[e] for e in range(q["E"])], DEV)
    ws = layer.MoEWorkspace(1, q["H"], q["I"], q["E"], 8, DEV)
    kept = []
    try:
        # step 0 is a prefill (T >= 2); decode steps take the bound launch
        x0 = synthetic.make_tokens(4, q["H"], seed=94)
        rt.forward(x0, layers[0].gate, layer=0, step=0)
        for step in range(1, 5):
            x = synthetic.make_tokens(1, q["H"], seed=94 + step)
            out, routing, row = rt.forward(x, layers[0].gate, layer=0, step=step)
            assert row["decode_path"] == "bound_launch"
            ref_out, logits, ids, w = layer.moe_forward(x, layers[0].gate, slots, ws, merge=rt.merge)
            torch.cuda.synchronize()
            assert torch.equal(out, ref_out) and torch.equal(routing.selected, ids.long())
            assert torch.equal(routing.logits, logits) and torch.equal(routing.weights, w)
            assert routing.selected.dtype == torch.int64 and routing.selected.shape == (1, 8)
            check_output(orc, out, routing, x, layers[0], q["H"], q["I"], 8, merge=rt.merge)
            kept.append((out, routing, ref_out.clone(), logits.clone(), ids.long(), w.clone()))
        torch.cuda.synchronize()
        for out, routing, ref_out, logits, ids, w in kept:
            assert torch.equal(out, ref_out) and torch.equal(routing.selected, ids)
            assert torch.equal(routing.logits, logits) and torch.equal(routing.weights, w)
        assert rt.bound_launches == 4 and len(rt._bindings) == 1
        closure(rt)
    finally:
        rt.close()


def test_runtime_bound_decode_across_the_launch_number_wrap(orc):
    """The bound launches are numbered 1 .. 32767 and the number wraps to 1:
    calls on both sides of the wrap (routed ids, prediction and error word
    all read back by their tags) still equal the single-launch layer and
    predict what the router picks for the next layer."""
    from pdscope_amd import layer, ops, synthetic
    from pdscope_amd.cache import ExpertKey
    from pdscope_amd.pdscope_runtime import PDScopeCudaRuntime
    q = synthetic.QWEN
    H, I, E, k = q["H"], q["I"], q["E"], q["k"]
    layers, masters = build(2, H, I, E, k, seed=193)
    hot = [ExpertKey(l, e, "bf16") for l in range(2) for e in range(E)]
    rt = PDScopeCudaRuntime(masters, hot_keys=hot, speculative_slots=0, resident_graphs=True)
    slots = ops.slot_table([layers[0].experts[e] for e in range(E)], DEV)
    ws = layer.MoEWorkspace(1, H, I, E, k, DEV)
    ws_pred = layer.MoEWorkspace(1, H, I, E, k, DEV)
    try:
        rt.forward(synthetic.make_tokens(4, H, seed=194), layers[0].gate, layer=0, step=0)
        rt._seq = 0x7FFF - 2
        seen = []
        for step in range(1, 6):
            x = synthetic.make_tokens(1, H, seed=194 + step)
            out, routing, row = rt.forward(x, layers[0].gate, layer=0, step=step, next_gate=layers[1].gate)
            seen.append(rt._seq)
            assert row["decode_path"] == "bound_launch"
            ref_out, logits, ids, w = layer.moe_forward(x, layers[0].gate, slots, ws, merge=rt.merge)
            _, _, pred, _ = layer.moe_forward(x, layers[1].gate, slots, ws_pred, merge=rt.merge)
            torch.cuda.synchronize()
            assert torch.equal(out, ref_out) and torch.equal(routing.selected, ids.long())
            assert torch.equal(routing.logits, logits) and torch.equal(routing.weights, w)
            got = rt._pinned_np[k:2 * k].tolist()
            assert sorted(v & 0xFFFF for v in got) == sorted(pred.view(-1).tolist())
            assert all(v >> 16 == rt._seq for v in got)
            check_output(orc, out, routing, x, layers[0], H, I, k, merge=rt.merge)
        assert seen == [0x7FFE, 0x7FFF, 1, 2, 3]
        closure(rt)
    finally:
        rt.close()


def test_runtime_prelaunches_a_fully_resident_prefill_layer(orc):
    """A prefill layer whose every expert has a ready copy is launched whole
    before its counts come back and its demand is revealed while it runs
    (decode_path 'prelaunched'): output and routing equal the resident layer
    (layer.moe_forward) bit for bit, the oracle holds, the ledger closes,
    and the prediction for the next layer is the router's.  A layer missing
    one copy takes the grouped path instead."""
    from pdscope_amd import layer, ops, synthetic
    from pdscope_amd.cache import ExpertKey
    from pdscope_amd.pdscope_runtime import PDScopeCudaRuntime
    H, I, E, k = 256, 128, 32, 4
    layers, masters = build(2, H, I, E, k, seed=83)
    hot = [ExpertKey(l, e, "bf16") for l in range(2) for e in range(E)]
    rt = PDScopeCudaRuntime(masters, hot_keys=hot, speculative_slots=0)
    slots = [ops.slot_table([layers[l].experts[e] for e in range(E)], DEV) for l in range(2)]
    ws = layer.MoEWorkspace(96, H, I, E, k, DEV)
    try:
        for i, T in enumerate((96, 17)):
            x = synthetic.make_tokens(T, H, seed=84 + i)
            for l in range(2):
                out, routing, row = rt.forward(x, layers[l].gate, layer=l, step=0, request=f"p{i}", top_k=k,
                                               next_gate=layers[1].gate if l == 0 else None)
                assert row["decode_path"] == "prelaunched"
                ref, _, ids, _ = layer.moe_forward(x, layers[l].gate, slots[l], ws, merge=rt.merge)
                torch.cuda.synchronize()
                assert torch.equal(out, ref) and torch.equal(routing.selected, ids.long()), (T, l)
                check_output(orc, out, routing, x, layers[l], H, I, k, merge=rt.merge)
                if l == 0:
                    _, nids, _ = layer.route(x, layers[1].gate, layer.MoEWorkspace(96, H, I, E, k, DEV))
                    torch.cuda.synchronize()
                    want = {}
                    for e in nids.reshape(-1).tolist():
                        want[e] = want.get(e, 0) + 1
                    assert row["next_prediction_counts"] == want
        closure(rt)
    finally:
        rt.close()
    # the Qwen shape at T=512, bitwise against the resident layer
    q = synthetic.QWEN
    qlayers, qmasters = build(1, q["H"], q["I"], q["E"], q["k"], seed=85)
    rt = PDScopeCudaRuntime(qmasters, hot_keys=[ExpertKey(0, e, "bf16") for e in range(q["E"])],
                            speculative_slots=0)
    try:
        x = synthetic.make_tokens(512, q["H"], seed=86)
        out, routing, row = rt.forward(x, qlayers[0].gate, layer=0, step=0)
        qws = layer.MoEWorkspace(512, q["H"], q["I"], q["E"], q["k"], DEV)
        qslots = ops.slot_table([qlayers[0].experts[e] for e in range(q["E"])], DEV)
        ref, _, ids, _ = layer.moe_forward(x, qlayers[0].gate, qslots, qws, merge=rt.merge)
        torch.cuda.synchronize()
        assert row["decode_path"] == "prelaunched"
        assert torch.equal(out, ref) and torch.equal(routing.selected, ids.long())
        closure(rt)
    finally:
        rt.close()
    # one expert without a copy: the grouped path after the reveal
    rt = PDScopeCudaRuntime(masters, hot_keys=hot[:E - 1], speculative_slots=0, demand_slots=2)
    try:
        x = synthetic.make_tokens(96, H, seed=87)
        out, routing, row = rt.forward(x, layers[0].gate, layer=0, step=0, top_k=k)
        torch.cuda.synchronize()
        assert row["decode_path"] == "grouped"
        check_output(orc, out, routing, x, layers[0], H, I, k, merge=rt.merge)
        closure(rt)
    finally:
        rt.close()


def test_runtime_raises_when_the_fused_decode_error_word_is_set():
    """The fused decode kernel sets a sticky error word when a bounded wait
    gives up.  Forced from the host here (the word is pre-set; the kernel only
    ever sets it), the runtime must raise on that layer call once the ledger
    has closed its demand, clear the word, and serve the next call normally."""
    from pdscope_amd import ops, synthetic
    from pdscope_amd.cache import ExpertKey
    from pdscope_amd.pdscope_runtime import PDScopeCudaRuntime
    q = synthetic.QWEN
    layers, masters = build(1, q["H"], q["I"], q["E"], q["k"], seed=97)
    hot = [ExpertKey(0, e, "bf16") for e in range(q["E"])]
    rt = PDScopeCudaRuntime(masters, hot_keys=hot, speculative_slots=0, resident_graphs=True)
    try:
        rt.forward(synthetic.make_tokens(4, q["H"], seed=98), layers[0].gate, layer=0, step=0)
        x = synthetic.make_tokens(1, q["H"], seed=99)
        out, _, row = rt.forward(x, layers[0].gate, layer=0, step=1)
        assert row["decode_path"] == "bound_launch"
        word = ops.decode_workspace(DEV, q["H"])
        word[ops.DECODE_WS_ERROR_WORD] = 1
        with pytest.raises(RuntimeError, match="bounded internal wait gave up"):
            rt.forward(x, layers[0].gate, layer=0, step=2)
        assert int(word[ops.DECODE_WS_ERROR_WORD].item()) == 0
        # the failed call closed its demand: the next token is served
        out3, _, row3 = rt.forward(x, layers[0].gate, layer=0, step=3)
        torch.cuda.synchronize()
        assert row3["decode_path"] == "bound_launch" and torch.equal(out3, out)
        closure(rt)
    finally:
        rt.close()
    # a fresh runtime on the same device serves normally after the cleared word
    rt = PDScopeCudaRuntime(masters, hot_keys=hot, speculative_slots=0, resident_graphs=True)
    try:
        rt.forward(synthetic.make_tokens(4, q["H"], seed=98), layers[0].gate, layer=0, step=0)
        out2, _, _ = rt.forward(x, layers[0].gate, layer=0, step=1)
        torch.cuda.synchronize()
        assert torch.equal(out, out2)
    finally:
        rt.close()


def test_runtime_partial_resident_bound_decode(orc):
    """Bound decode launch over a partly resident layer: experts without a copy
    read as null on the first launch; misses are staged in one batch and the
    layer is launched again over the completed table.  The output equals the
    single-launch layer over a fully resident table bit for bit; the
    predictor prefetches the next layer's experts on the way."""
    from pdscope_amd import layer, ops, synthetic
    from pdscope_amd.cache import ExpertKey
    from pdscope_amd.pdscope_runtime import PDScopeCudaRuntime
    q = synthetic.QWEN
    layers, masters = build(2, q["H"], q["I"], q["E"], q["k"], seed=95)
    hot = [ExpertKey(l, e, "bf16") for l in range(2) for e in range(32)]
    rt = PDScopeCudaRuntime(masters, hot_keys=hot, speculative_slots=8, demand_slots=8, resident_graphs=True)
    full = [ops.slot_table([layers[l].experts[e] for e in range(q["E"])], DEV) for l in range(2)]
    ws = layer.MoEWorkspace(1, q["H"], q["I"], q["E"], 8, DEV)
    misses = 0
    try:
        x0 = synthetic.make_tokens(4, q["H"], seed=96)
        for l in range(2):
            rt.forward(x0, layers[l].gate, layer=l, step=0, next_gate=layers[1].gate if l == 0 else None)
        for step in range(1, 6):
            x = synthetic.make_tokens(1, q["H"], seed=96 + step)
            for l in range(2):
                out, routing, row = rt.forward(x, layers[l].gate, layer=l, step=step,
                                               next_gate=layers[1].gate if l == 0 else None)
                assert row["decode_path"] == "bound_launch"
                misses += len(row["decision"]["on_demand_queue"])
                ref_out, _, ids, _ = layer.moe_forward(x, layers[l].gate, full[l], ws, merge=rt.merge)
                torch.cuda.synchronize()
                assert torch.equal(routing.selected, ids.long())
                assert torch.equal(out, ref_out)
                check_output(orc, out, routing, x, layers[l], q["H"], q["I"], 8, merge=rt.merge)
                if l == 0:
                    # the prediction the bound launch made equals the router on the next gate
                    nids = torch.empty((1, 8), dtype=torch.int32, device=DEV)
                    ops.route_topk(x, layers[1].gate, 8, True,
                                   out=(torch.empty((1, q["E"]), dtype=torch.bfloat16, device=DEV), nids,
                                        torch.empty((1, 8), dtype=torch.bfloat16, device=DEV)))
                    torch.cuda.synchronize()
                    assert row["next_prediction_counts"] == {int(e): 1 for e in nids[0].tolist()}
        assert misses > 0
        closure(rt)
        assert rt.cache.stats().get("prefetch_loads_submitted", 0) > 0
    finally:
        rt.close()


def test_runtime_rejects_bad_phase_shapes():
    from pdscope_amd.cache import ExpertKey
    from pdscope_amd.pdscope_runtime import PDScopeCudaRuntime
    layers, masters = build(1, 256, 128, 32, 4)
    rt = PDScopeCudaRuntime(masters, hot_keys=[ExpertKey(0, 0, "bf16")], speculative_slots=0)
    try:
        x1 = torch.zeros((1, 256), dtype=torch.bfloat16, device=DEV)
        x2 = torch.zeros((2, 256), dtype=torch.bfloat16, device=DEV)
        with pytest.raises(ValueError):
            rt.forward(x1, layers[0].gate, layer=0, step=0)
        with pytest.raises(ValueError):
            rt.forward(x2, layers[0].gate, layer=0, step=1)
        with pytest.raises(ValueError):
            rt.forward(x2, layers[0].gate, layer=5, step=0)
        with pytest.raises(ValueError):   # hidden size of another model
            rt.forward(torch.zeros((2, 128), dtype=torch.bfloat16, device=DEV), layers[0].gate, layer=0, step=0)
        with pytest.raises(ValueError):   # gate of another shape
            rt.forward(x2, layers[0].gate[:16], layer=0, step=0)
    finally:
        rt.close()
    with pytest.raises(ValueError):
        PDScopeCudaRuntime(masters, hot_keys=[], speculative_slots=0, demand_slots=1)


def test_executor_per_expert_hook_matches_oracle(orc):
    from pdscope_amd.cache import DemandID, ExpertCache, ExpertKey
    from pdscope_amd.executor import ExpertExecutor
    H, I, E, k = 256, 128, 32, 4
    layers, masters = build(1, H, I, E, k, seed=5)
    sizes = {key: w.nbytes for key, w in masters.items()}
    size = next(iter(sizes.values()))
    cache = ExpertCache(sizes, 4 * size, [size, size])
    ex = ExpertExecutor(cache, masters, 0)
    try:
        key = ExpertKey(0, 3, "bf16")
        cache.on_demand(DemandID("r", 0, 0), {key: 7})
        t = ex.load(key)
        assert ex.finish_load(t, wait=True)
        x = torch.randn((7, H), device=DEV).to(torch.bfloat16)
        pend = ex.gpu(key, x)
        y = ex.finish_gpu(pend, wait=True)
        blk = u16(layers[0].experts[3])
        ref = orc.expert_forward(u16(x), blk[:I * H].reshape(I, H), blk[I * H:2 * I * H].reshape(I, H),
                                 blk[2 * I * H:].reshape(H, I))
        assert_layer_close(orc, y, ref)
        cache.end_demand(DemandID("r", 0, 0))
        # the staged bytes equal the pinned master bytes
        flat = ex.copies[t]
        assert torch.equal(flat.cpu(), masters[key].flat.view(torch.uint8))
    finally:
        ex.shutdown()


def test_executor_accounts_an_enqueued_use_only_after_it_completed():
    """gpu_group(launch=None) accounts uses that work enqueued before the
    reveal already made: without a completed event recorded after that work
    it raises and acquires nothing; with one it holds the copies until its
    own event on that stream completes, then finish_gpu releases them."""
    from pdscope_amd.cache import DemandID, ExpertCache, ExpertKey
    from pdscope_amd.executor import ExpertExecutor
    H, I, E, k = 256, 128, 32, 4
    _, masters = build(1, H, I, E, k, seed=6)
    sizes = {key: w.nbytes for key, w in masters.items()}
    size = next(iter(sizes.values()))
    cache = ExpertCache(sizes, 4 * size, [size, size])
    ex = ExpertExecutor(cache, masters, 0)
    try:
        key = ExpertKey(0, 5, "bf16")
        cache.on_demand(DemandID("r", 0, 0), {key: 1})
        assert ex.finish_load(ex.load(key), wait=True)
        cur = torch.cuda.current_stream()
        with pytest.raises(RuntimeError, match="completed"):
            ex.gpu_group([key], None, wait_for=cur)
        assert not ex.computes
        done = torch.cuda.Event()
        done.record(cur)
        done.synchronize()
        pend = ex.gpu_group([key], None, wait_for=cur, completed=done)
        assert ex.computes and ex.finish_gpu(pend, wait=True) is None and not ex.computes
        cache.end_demand(DemandID("r", 0, 0))
    finally:
        ex.shutdown()


def test_executor_holds_a_running_use_until_its_proof_completes():
    """gpu_group(launch=None, running=proof) holds the copies of work that
    may still run: finish_gpu(wait=False) leaves them held while the proof
    reports the work running, finish_gpu(wait=True) waits through the
    proof's synchronize() and then releases them; a call names exactly one
    of completed= and running=, and the proof never joins the executor's
    event pool."""
    from pdscope_amd.cache import DemandID, ExpertCache, ExpertKey
    from pdscope_amd.executor import ExpertExecutor
    H, I, E, k = 256, 128, 32, 4
    _, masters = build(1, H, I, E, k, seed=7)
    sizes = {key: w.nbytes for key, w in masters.items()}
    size = next(iter(sizes.values()))
    cache = ExpertCache(sizes, 4 * size, [size, size])
    ex = ExpertExecutor(cache, masters, 0)

    class Proof:   # a completion proof the test flips by hand
        def __init__(self):
            self.done, self.waited = False, 0

        def query(self):
            return self.done

        def synchronize(self):
            self.waited += 1
            self.done = True

    try:
        key = ExpertKey(0, 3, "bf16")
        ident = DemandID("r", 0, 0)
        cache.on_demand(ident, {key: 1})
        assert ex.finish_load(ex.load(key), wait=True)
        cur = torch.cuda.current_stream()
        proof = Proof()
        with pytest.raises(RuntimeError, match="exactly one"):
            ex.gpu_group([key], None, wait_for=cur, completed=proof, running=proof)
        assert not ex.computes
        pend = ex.gpu_group([key], None, wait_for=cur, running=proof)
        assert cache.lookup(key).state == "in_use"
        assert ex.finish_gpu(pend) is None and ex.computes and cache.lookup(key).state == "in_use"
        assert ex.finish_gpu(pend, wait=True) is None and not ex.computes
        assert proof.waited == 1 and cache.lookup(key).state == "ready"
        assert all(e is not proof for e in ex._free_events)
        cache.end_demand(ident)
    finally:
        ex.shutdown()


def test_executor_profiles_stages_and_stages_masters_by_memcpy(orc):
    """profile_stages records the copy, launch and CPU-call spans
    (expertbench/executor.py:352-355, 384-385, 472-481, 518-528); lazily
    pinned masters copied byte for byte (cpu_staging_copy="memcpy") stage the
    same bytes; a callable CPU backend runs on an initialised worker."""
    from pdscope_amd.cache import DemandID, ExpertCache, ExpertKey
    from pdscope_amd.executor import ExpertExecutor
    from pdscope_amd import synthetic
    from pdscope_amd.executor import masters_from_block
    H, I, E, k = 256, 128, 32, 4
    layers = [synthetic.make_layer(H, I, E, k, True, seed=11, device=DEV)]
    masters = masters_from_block(0, layers[0].experts, E, H, I, pin=False)   # pinned on first use
    sizes = {key: w.nbytes for key, w in masters.items()}
    size = next(iter(sizes.values()))
    cache = ExpertCache(sizes, 4 * size, [size, size])

    def cpu_expert(key, rows):
        return torch.zeros_like(rows)
    ex = ExpertExecutor(cache, masters, 0, profile_stages=True, pinned_source_mode="lazy_pinned",
                        cpu_staging_copy="memcpy", cpu_backend=cpu_expert)
    try:
        key, cpu_key = ExpertKey(0, 9, "bf16"), ExpertKey(0, 2, "bf16")
        cache.on_demand(DemandID("r", 0, 0), {key: 3, cpu_key: 2})
        t = ex.load(key)
        assert ex.finish_load(t, wait=True)
        st = ex.stage_timings
        assert st["weight_dma_gpu_span_ms"] > 0 and st["source_copy_ms"] > 0
        assert torch.equal(ex.copies[t].cpu(), masters[key].flat.view(torch.uint8))
        x = torch.randn((3, H), device=DEV).to(torch.bfloat16)
        y = ex.finish_gpu(ex.gpu(key, x), wait=True)
        blk = u16(layers[0].experts[9])
        ref = orc.expert_forward(u16(x), blk[:I * H].reshape(I, H), blk[I * H:2 * I * H].reshape(I, H),
                                 blk[2 * I * H:].reshape(H, I))
        assert_layer_close(orc, y, ref)
        assert st["gpu_forward_device_span_ms"] > 0 and st["gpu_forward_host_submit_ms"] >= 0
        rows = torch.randn((2, H)).to(torch.bfloat16)
        out = ex.finish_cpu(ex.submit_cpu(cpu_key, rows), wait=True)
        assert out.shape == rows.shape and st["cpu_forward_ms"] >= 0
        assert ex.cpu_worker_init["torch_threads"] == ex.cpu_worker_init["expected_threads"]
        cache.end_demand(DemandID("r", 0, 0))
    finally:
        ex.shutdown()


def test_executor_slot_table_upload_follows_the_host_mirror():
    """upload_table copies a layer's table again only after an entry changed;
    every upload, skipped or not, leaves the device table equal to the host
    mirror as seen from the stream that asked for it."""
    from pdscope_amd.cache import DemandID, ExpertCache, ExpertKey
    from pdscope_amd.executor import ExpertExecutor
    H, I, E, k = 256, 128, 32, 4
    _, masters = build(1, H, I, E, k, seed=6)
    sizes = {key: w.nbytes for key, w in masters.items()}
    size = next(iter(sizes.values()))
    cache = ExpertCache(sizes, 4 * size, [size, size])
    ex = ExpertExecutor(cache, masters, 0)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()

    def device_table(stream):
        dev = ex.upload_table(0, E, stream)
        with torch.cuda.stream(stream):
            snap = dev.clone()
        stream.synchronize()
        return snap.cpu().tolist()

    try:
        assert device_table(s1) == [0] * E
        copies_before = ex._ring.i
        assert device_table(s2) == [0] * E          # unchanged: no new copy
        assert ex._ring.i == copies_before
        key = ExpertKey(0, 3, "bf16")
        cache.on_demand(DemandID("r", 1, 0), {key: 1})
        t = ex.load(key)
        assert ex.finish_load(t, wait=True)
        want = [0] * E
        want[3] = ex.copies[t].data_ptr()
        assert ex.table(0, E)[1] == want
        assert device_table(s2) == want             # changed: copied again
        assert ex._ring.i != copies_before
        assert device_table(s1) == want             # unchanged, read from the other stream
    finally:
        ex.shutdown()


class _Pool:
    def __init__(self):
        self.q = []

    def submit(self, task):
        self.q.append(task)

    def sync(self):
        for t in self.q:
            t()
        self.q.clear()


class _OracleLayer:
    """CPU expert queue layer: forward_task runs the oracle expert per packed row."""

    def __init__(self, orc, experts_u16, H, I):
        self.orc, self.experts, self.H, self.I = orc, experts_u16, H, I

    def forward_task(self, count_ptr, k, selected_ptr, coeff_ptr, in_ptr, out_ptr, flag):
        def run():
            n = ctypes.c_int32.from_address(count_ptr).value
            sel = np.ctypeslib.as_array((ctypes.c_int64 * n).from_address(selected_ptr))
            x = np.ctypeslib.as_array((ctypes.c_uint16 * (n * self.H)).from_address(in_ptr)).reshape(n, self.H)
            out = np.ctypeslib.as_array((ctypes.c_uint16 * (n * self.H)).from_address(out_ptr)).reshape(n, self.H)
            IH = self.I * self.H
            for r in range(n):
                blk = self.experts[sel[r]]
                out[r] = self.orc.expert_forward(x[r:r + 1].copy(), blk[:IH].reshape(self.I, self.H),
                                                 blk[IH:2 * IH].reshape(self.I, self.H),
                                                 blk[2 * IH:].reshape(self.H, self.I))[0]
        return run


@pytest.fixture(params=["package", "reference_loader"])
def nd(request, dispatch_via_reference_loader):
    """The pdscope_layer_dispatch extension as the package imports it and as
    the reference driver's loader finds it."""
    if request.param == "package":
        from pdscope_amd import pdscope_layer_dispatch
        return pdscope_layer_dispatch
    return dispatch_via_reference_loader


def test_native_dispatch_submit_and_merge(orc, nd):
    H, I, E, k = 256, 128, 32, 4
    layers, _ = build(1, H, I, E, k, seed=8)
    experts = u16(layers[0].experts)
    rows = 3
    ids = [5, 17, 2]
    row = torch.randn(H).to(torch.bfloat16)
    packed = torch.empty((rows, H), dtype=torch.bfloat16)
    block = torch.empty((rows, H), dtype=torch.bfloat16)
    count, sel, coeff = ctypes.c_int32(0), (ctypes.c_int64 * rows)(), (ctypes.c_float * rows)()
    scratch = torch.empty((rows, H), dtype=torch.bfloat16, device=DEV)
    out = torch.zeros((1, H), dtype=torch.bfloat16, device=DEV)
    tokens = torch.zeros(rows, dtype=torch.long, device=DEV)
    weights = torch.tensor([0.5, 0.25, 0.125], dtype=torch.bfloat16, device=DEV)
    res = nd.submit_and_merge(_Pool(), _OracleLayer(orc, experts, H, I), row.data_ptr(), rows, H * 2,
                              packed.data_ptr(), block.data_ptr(), scratch, ctypes.addressof(count),
                              ctypes.addressof(sel), ctypes.addressof(coeff), ids, out, tokens, weights)
    torch.cuda.synchronize()
    assert res is out
    ref = torch.zeros(H, dtype=torch.bfloat16)
    for r in range(rows):
        ref = (ref.float() + (block[r] * weights.cpu()[r]).float()).to(torch.bfloat16)
    assert torch.equal(out.cpu()[0], ref)


def test_native_dispatch_submit_then_finish_and_merge_with_an_out_of_range_token(orc, nd):
    """submit_group then finish_and_merge (the split form the runtime uses);
    a token index outside out's rows is skipped by the merge, every other
    row is added in order with bf16 arithmetic."""
    H, I, E, k = 256, 128, 32, 4
    layers, _ = build(1, H, I, E, k, seed=9)
    experts = u16(layers[0].experts)
    rows, ids = 4, [3, 30, 8, 11]
    row = torch.randn(H).to(torch.bfloat16)
    packed = torch.empty((rows, H), dtype=torch.bfloat16)
    block = torch.empty((rows, H), dtype=torch.bfloat16)
    count, sel, coeff = ctypes.c_int32(0), (ctypes.c_int64 * rows)(), (ctypes.c_float * rows)()
    scratch = torch.empty((rows, H), dtype=torch.bfloat16, device=DEV)
    base = torch.randn((2, H)).to(torch.bfloat16)
    out = base.to(DEV)
    tokens = torch.tensor([1, 7, 0, 1], dtype=torch.long, device=DEV)   # 7 is past out's 2 rows
    weights = torch.tensor([0.5, 4.0, -0.25, 0.125], dtype=torch.bfloat16, device=DEV)
    pool = _Pool()
    nd.submit_group(pool, _OracleLayer(orc, experts, H, I), row.data_ptr(), rows, H * 2, packed.data_ptr(),
                    block.data_ptr(), ctypes.addressof(count), ctypes.addressof(sel), ctypes.addressof(coeff), ids)
    res = nd.finish_and_merge(pool, block.data_ptr(), rows, H * 2, scratch, out, tokens, weights)
    torch.cuda.synchronize()
    assert res is out and list(sel) == ids
    ref = base.clone()
    for r, t in enumerate([1, 7, 0, 1]):
        if t < 2:
            ref[t] = (ref[t].float() + (block[r] * weights.cpu()[r]).float()).to(torch.bfloat16)
    assert torch.equal(out.cpu(), ref)
