"""Host half of the native dispatch (CPU only): packing and the queue protocol.

The pdscope_layer_dispatch extension is exercised both as the package's
module and as the reference driver's loader finds it (glob under
expertbench/native-build/layer-dispatch, spec_from_file_location,
exec_module)."""
import ctypes
from pathlib import Path

import pytest
import torch


class FakePool:
    def __init__(self):
        self.queue, self.synced = [], 0

    def submit(self, task):
        self.queue.append(task)

    def sync(self):
        for t in self.queue:
            t()
        self.queue.clear()
        self.synced += 1


class RecordingLayer:
    def __init__(self):
        self.calls = []

    def forward_task(self, count_ptr, k, selected_ptr, coeff_ptr, in_ptr, out_ptr, flag):
        self.calls.append((count_ptr, k, selected_ptr, coeff_ptr, in_ptr, out_ptr, flag))
        return lambda: None


@pytest.fixture(params=["package", "reference_loader"])
def nd(request, dispatch_via_reference_loader):
    if request.param == "package":
        from pdscope_amd import pdscope_layer_dispatch
        return pdscope_layer_dispatch
    return dispatch_via_reference_loader


def test_module_is_the_native_extension(nd):
    from pdscope_amd import build as B
    assert Path(nd.__file__).resolve() == B.DISPATCH_MODULE.resolve()
    assert nd.__file__.endswith(".so") and all(callable(getattr(nd, f)) for f in
                                               ("submit_group", "finish_and_merge", "submit_and_merge"))


def test_submit_group_packs_rows_ids_and_unit_coefficients(nd):
    rows, H = 5, 64
    row = torch.randn(H).to(torch.bfloat16)
    packed = torch.empty((rows, H), dtype=torch.bfloat16)
    block = torch.empty((rows, H), dtype=torch.bfloat16)
    count = ctypes.c_int32(0)
    selected = (ctypes.c_int64 * rows)()
    coeff = (ctypes.c_float * rows)()
    pool, layer = FakePool(), RecordingLayer()
    ids = [7, 3, 11, 0, 42]
    nd.submit_group(pool, layer, row.data_ptr(), rows, H * 2, packed.data_ptr(), block.data_ptr(),
                    ctypes.addressof(count), ctypes.addressof(selected), ctypes.addressof(coeff), ids)
    assert count.value == rows and list(selected) == ids and list(coeff) == [1.0] * rows
    assert torch.equal(packed, row.expand(rows, H))
    assert len(pool.queue) == 1 and pool.synced == 0           # submitted, not joined
    c = layer.calls[0]
    assert c[1] == 1 and c[6] is False and c[4] == packed.data_ptr() and c[5] == block.data_ptr()


@pytest.mark.parametrize("rows,row_bytes,ids", [(0, 4096, []), (2, 3, [1, 2]), (2, 4096, [1])])
def test_submit_group_rejects_bad_shapes(nd, rows, row_bytes, ids):
    with pytest.raises(RuntimeError):
        nd.submit_group(FakePool(), RecordingLayer(), 1, rows, row_bytes, 1, 1, 1, 1, 1, ids)


def test_finish_and_merge_rejects_host_tensors(nd):
    t = torch.zeros(4, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError):
        nd.finish_and_merge(FakePool(), 1, 1, 8, t, t, torch.zeros(1, dtype=torch.long), t)


def test_submit_and_merge_rejects_host_tensors_before_submitting(nd):
    pool = FakePool()
    t = torch.zeros(4, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="CUDA device"):
        nd.submit_and_merge(pool, RecordingLayer(), 1, 1, 8, 1, 1, t, 1, 1, 1, [3], t,
                            torch.zeros(1, dtype=torch.long), t)
    assert pool.queue == [] and pool.synced == 0


def test_layer_and_pool_errors_propagate(nd):
    class Broken:
        def forward_task(self, *args):
            raise KeyError("no such expert layer")
    rows, H = 2, 64
    row = torch.zeros(H, dtype=torch.bfloat16)
    packed = torch.empty((rows, H), dtype=torch.bfloat16)
    count, selected, coeff = ctypes.c_int32(0), (ctypes.c_int64 * rows)(), (ctypes.c_float * rows)()
    with pytest.raises(KeyError):
        nd.submit_group(FakePool(), Broken(), row.data_ptr(), rows, H * 2, packed.data_ptr(), packed.data_ptr(),
                        ctypes.addressof(count), ctypes.addressof(selected), ctypes.addressof(coeff), [1, 2])
