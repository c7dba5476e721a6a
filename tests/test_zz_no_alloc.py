"""GPU test of pdscope_pack_static, the grouping entry point that allocates
nothing: its outputs must equal pdscope_pack's (with a caller workspace) bit
for bit, on successive calls that reuse the library-owned scratch with a
smaller input the second time, and when captured in a hipGraph and replayed
over new ids in the same buffers; it must refuse inputs above its limit
before launching anything."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ids(T, k, E, seed, skew=False):
    g = torch.Generator().manual_seed(seed)
    if skew:
        p = torch.arange(1, E + 1, dtype=torch.float64) ** -1.1
        rows = [torch.multinomial(p, k, replacement=False, generator=g) for _ in range(T)]
        ids = torch.stack(rows)
    else:
        ids = torch.argsort(torch.rand(T, E, generator=g), dim=1)[:, :k]
    return ids.to(torch.int32).to(DEV).contiguous()


def _buffers(T, k, E, fill):
    n = T * k
    mk = lambda m: torch.full((m,), fill, dtype=torch.int32, device=DEV)  # noqa: E731
    from pdscope_amd import ops
    return ops.Packed(mk(E), mk(E + 1), mk(n), mk(n), mk(n))


def _same(a, b):
    for name in ("counts", "offsets", "perm_token", "perm_pos", "row_of"):
        x, y = getattr(a, name).cpu().numpy(), getattr(b, name).cpu().numpy()
        assert np.array_equal(x, y), f"{name} differs"


def test_pack_static_equals_pack_on_successive_calls():
    from pdscope_amd import ops
    cases = [(4096, 8, 128, False), (1000, 6, 64, True), (16, 8, 128, False), (2600, 8, 128, True)]
    for i, (T, k, E, skew) in enumerate(cases):
        print(f"pack_static case {i}: T={T} k={k} E={E} skew={skew}", flush=True)
        ids = _ids(T, k, E, seed=100 + i, skew=skew)
        want = ops.pack(ids, E)
        got = ops.pack_static(ids, E, _buffers(T, k, E, fill=-7))
        torch.cuda.synchronize()
        _same(got, want)
        assert int(got.offsets[E].item()) == T * k


def test_pack_static_refuses_inputs_above_its_limit():
    from pdscope_amd import ops
    limit = ops.pack_static_max_ids()
    assert limit == 1 << 20
    T, k, E = limit // 8 + 1, 8, 128
    ids = torch.zeros((T, k), dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError, match="static scratch limit"):
        ops.pack_static(ids, E, _buffers(T, k, E, fill=0))


def test_pack_static_replays_in_a_captured_graph():
    """The multi-block path (T*k > 2048) captured once in a hipGraph after
    the set-up lookup, then replayed over new ids copied into the same
    buffer, with eager work between replays: every replay equals pdscope_pack
    on those ids bit for bit."""
    from pdscope_amd import ops
    T, k, E = 4096, 8, 128
    assert ops.pack_static_max_ids() == 1 << 20    # set-up: the scratch lookup, outside the capture
    ids_buf = _ids(T, k, E, seed=200)
    out = _buffers(T, k, E, fill=-7)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ops.pack_static(ids_buf, E, out)            # eager warm-up on a side stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.pack_static(ids_buf, E, out)
    for i, skew in enumerate([False, True, False, True]):
        print(f"pack_static graph replay {i}: T={T} k={k} E={E} skew={skew}", flush=True)
        new = _ids(T, k, E, seed=300 + i, skew=skew)
        ids_buf.copy_(new)
        want = ops.pack(new, E)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        _same(out, want)
