"""Native decode MoE tail: submit, join, stage and merge (the ``pdscope_layer_dispatch`` module).

Same entry points, argument meaning and errors as
native/native_layer_dispatch.cpp:49-142:

* ``submit_group(pool, layer, row_ptr, rows, row_bytes, packed_ptr, block_ptr,
  count_ptr, selected_ptr, coeff_ptr, ids)`` packs ``rows`` copies of one
  activation row with their expert ids (pdscope_dispatch_pack, native) and
  submits ONE ``layer.forward_task(count, 1, selected, coeff, packed, block,
  False)`` to the CPU expert queue ``pool`` without joining it;
* ``finish_and_merge(pool, block_ptr, rows, row_bytes, scratch, out, tokens,
  weights)`` joins the queue, copies the CPU block into device ``scratch`` on
  the current stream and adds ``scratch * weights`` into ``out`` at ``tokens``
  (pdscope_stage_merge: bf16 arithmetic, rows in order); returns ``out``;
* ``submit_and_merge(...)`` does both in one call.

``pool`` (submit/sync) and ``layer`` (forward_task) are the caller's CPU
expert queue objects, used exactly as the reference uses them.  Shape and
device errors raise RuntimeError as the reference's std::runtime_error does.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .ops import stage_merge


def _pack(row_ptr, rows, row_bytes, packed_ptr, count_ptr, selected_ptr, coeff_ptr, ids):
    if rows < 1 or row_bytes < 2 or row_bytes % 2 != 0:
        raise RuntimeError("invalid decode pack shape")
    if len(ids) != rows:
        raise RuntimeError("expert id count must match the packed row count")
    arr = (ctypes.c_int64 * rows)(*ids)
    try:
        _lib.call("pdscope_dispatch_pack", ctypes.c_void_p(int(row_ptr)), int(rows), int(row_bytes),
                  ctypes.c_void_p(int(packed_ptr)), ctypes.c_void_p(int(count_ptr)),
                  ctypes.c_void_p(int(selected_ptr)), ctypes.c_void_p(int(coeff_ptr)), arr)
    except ValueError as err:
        raise RuntimeError(str(err)) from None


def submit_group(pool, layer, row_ptr, rows, row_bytes, packed_ptr, block_ptr, count_ptr, selected_ptr, coeff_ptr,
                 ids):
    """Pack and submit the decode CPU group to the native queue without joining it."""
    _pack(row_ptr, rows, row_bytes, packed_ptr, count_ptr, selected_ptr, coeff_ptr, list(ids))
    task = layer.forward_task(count_ptr, 1, selected_ptr, coeff_ptr, packed_ptr, block_ptr, False)
    pool.submit(task)


def _check_device(scratch, out, tokens, weights):
    if not (scratch.is_cuda and out.is_cuda and tokens.is_cuda and weights.is_cuda):
        raise RuntimeError("scratch/out/tokens/weights must live on the CUDA device")


def finish_and_merge(pool, block_ptr, rows, row_bytes, scratch, out, tokens, weights):
    """Join the native queue, stage the packed block and scatter it into the output."""
    _check_device(scratch, out, tokens, weights)
    pool.sync()
    if scratch.numel() * scratch.element_size() != rows * row_bytes:
        raise RuntimeError("scratch buffer must match the packed block")
    stage_merge(int(block_ptr), int(rows), int(row_bytes), scratch, out, tokens.contiguous(),
                weights.to(torch.bfloat16).contiguous())
    return out


def submit_and_merge(pool, layer, row_ptr, rows, row_bytes, packed_ptr, block_ptr, scratch, count_ptr,
                     selected_ptr, coeff_ptr, ids, out, tokens, weights):
    """Native decode MoE tail: submit, join, stage and merge in one call."""
    if rows < 1 or row_bytes < 2 or row_bytes % 2 != 0:
        raise RuntimeError("invalid decode pack shape")
    if len(ids) != rows:
        raise RuntimeError("expert id count must match the packed row count")
    _check_device(scratch, out, tokens, weights)
    submit_group(pool, layer, row_ptr, rows, row_bytes, packed_ptr, block_ptr, count_ptr, selected_ptr, coeff_ptr,
                 ids)
    return finish_and_merge(pool, block_ptr, rows, row_bytes, scratch, out, tokens, weights)
