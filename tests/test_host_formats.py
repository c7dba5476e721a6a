"""Host-side formats and cost views (CPU only): the static hot profile, private
master copies and the resident-graph cost view of a cost table."""
import json
import math

import pytest
import torch

from pdscope_amd.cache import ExpertKey
from pdscope_amd.checkpoint import copy_cpu_master_storage
from pdscope_amd.costs import FileCosts, ResidentGraphCosts
from pdscope_amd.executor import ExpertWeights
from pdscope_amd.pdscope_runtime import load_hot_profile

K = lambda l, e: ExpertKey(l, e, "bf16")  # noqa: E731


def _masters(n_layers=2, E=4, H=16, I=8):
    g = torch.Generator().manual_seed(1)
    out = {}
    for l in range(n_layers):
        for e in range(E):
            t = {p: torch.randn(s, generator=g).to(torch.bfloat16)
                 for p, s in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I)))}
            out[K(l, e)] = ExpertWeights(K(l, e), t, {"source": "test"})
    return out


def test_hot_profile_selects_listed_experts_in_file_order(tmp_path):
    masters = _masters()
    p = tmp_path / "hot.txt"
    p.write_text("1,2\n\n0,3\n5,0\n0,1\n")          # (5,0) has no master
    keys, info = load_hot_profile(p, masters, 3)
    assert keys == [K(1, 2), K(0, 3), K(0, 1)]
    assert info["entries"] == 4 and info["eligible_entries"] == 3 and info["selected"] == 3
    assert len(info["sha256"]) == 64
    keys, _ = load_hot_profile(p, masters, 1)
    assert keys == [K(1, 2)]


@pytest.mark.parametrize("text,slots", [("0,1\n0,1\n", 1), ("0,1,2\n", 1), ("0;1\n", 1), ("-1,0\n", 1),
                                        ("0,1\n", 2), ("0,1\n", -1), ("0,1\n", 1.0)])
def test_hot_profile_refusals(tmp_path, text, slots):
    p = tmp_path / "hot.txt"
    p.write_text(text)
    with pytest.raises(ValueError):
        load_hot_profile(p, _masters(), slots)


def test_private_master_copies_own_their_storage():
    masters = _masters()
    before = {k: {p: t.clone() for p, t in w.tensors.items()} for k, w in masters.items()}
    ptrs = {k: w.tensors["up_proj"].data_ptr() for k, w in masters.items()}
    info = copy_cpu_master_storage(masters)
    assert info["experts_copied"] == len(masters)
    assert info["bytes_copied"] == sum(w.nbytes for w in masters.values())
    for k, w in masters.items():
        assert w.tensors["up_proj"].data_ptr() != ptrs[k]
        assert all(torch.equal(w.tensors[p], before[k][p]) for p in before[k])
        assert w.provenance["storage"] == "private CPU copy"


def test_resident_graph_costs_closed_form(tmp_path):
    pts = {n: dict(cpu_ms=0.3 * n, gpu_ms=0.2 + 0.001 * n, h2d_ms=0.9 + 0.001 * n)
           for n in (1, 4, 16, 64, 128, 256, 1024, 4096)}
    path = tmp_path / "c.json"
    path.write_text(json.dumps(dict(kind="pdscope_cost_table", points={str(n): p for n, p in pts.items()})))
    base = FileCosts(path)
    eager = ResidentGraphCosts(base, 0.05, "eager_bound")
    measured = ResidentGraphCosts(base, 0.05, "measured")
    assert eager.for_load(1) == base.for_load(1)
    one = measured.for_load(1)
    # one-token GPU work at the replay cost; copy + compute of a staged expert unchanged
    assert one["gpu_ms"] == 0.05 and math.isclose(one["h2d_ms"] + one["gpu_ms"], pts[1]["h2d_ms"] + pts[1]["gpu_ms"])
    assert measured.for_load(64) == base.for_load(64)
    assert measured.sources == base.sources
    tiny = ResidentGraphCosts(base, 10.0, "measured").for_load(1)
    assert tiny["h2d_ms"] == 1e-6                      # never a non-positive copy time
    for bad in (("eager_bound", 0.0), ("other", 0.1)):
        with pytest.raises(ValueError):
            ResidentGraphCosts(base, bad[1], bad[0])


def test_decode_error_word_raises_and_is_cleared():
    """The runtime's check of the fused decode kernel's sticky error word, on
    the CPU: a zero word passes, a set word raises for that call and is
    cleared, so the next call reports only its own."""
    from pdscope_amd.pdscope_runtime import PDScopeCudaRuntime
    word = torch.zeros(1, dtype=torch.int32)

    class Holder:
        def _decode_error_word(self):
            return word

    h = Holder()
    PDScopeCudaRuntime._raise_if_decode_gave_up(h, 0)
    word[0] = 1
    with pytest.raises(RuntimeError, match="bounded internal wait gave up"):
        PDScopeCudaRuntime._raise_if_decode_gave_up(h, int(word[0]))
    assert int(word[0]) == 0
    PDScopeCudaRuntime._raise_if_decode_gave_up(h, int(word[0]))
