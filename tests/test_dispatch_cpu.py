"""Host half of the native dispatch (CPU only): packing and the queue protocol."""
import ctypes

import numpy as np
import pytest
import torch

from pdscope_amd import pdscope_layer_dispatch as nd


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


def test_submit_group_packs_rows_ids_and_unit_coefficients():
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
def test_submit_group_rejects_bad_shapes(rows, row_bytes, ids):
    with pytest.raises(RuntimeError):
        nd.submit_group(FakePool(), RecordingLayer(), 1, rows, row_bytes, 1, 1, 1, 1, 1, ids)


def test_finish_and_merge_rejects_host_tensors():
    t = torch.zeros(4, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError):
        nd.finish_and_merge(FakePool(), 1, 1, 8, t, t, torch.zeros(1, dtype=torch.long), t)
