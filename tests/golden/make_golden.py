"""Write the golden fixtures that pin the C oracle.

The reference ships no golden vectors (its checks are runtime assertions on
real Qwen3 weights that are not available here).  These fixtures are produced
by an independent torch-CPU restatement of the reference formulas, written
line by line from the cited sources, so the C oracle can be checked against
the same library arithmetic the reference uses (torch 2.10):

* route           expertbench/adapters/qwen.py:140-152, with the lower-index
                  tie rule made explicit by a stable descending sort
                  (torch.topk leaves tie order unspecified);
* compact groups  expertbench/pdscope_runtime.py:16-39 (stable argsort of the
                  slot-major flat ids);
* expert groups   expertbench/adapters/qwen.py:155-174 (torch.where over the
                  transposed expert mask) -- a second, independent grouping;
* expert_forward  expertbench/adapters/qwen.py:87-90 on CPU bf16 tensors and
                  reference_fp32 qwen.py:93-98;
* merge           the default merge='reference' of
                  expertbench/pdscope_runtime.py:454-468 (zero output, one bf16
                  index_add_ of parts[e] * coeff per expert, experts ascending);
* native tail     the out.index_add_(0, tokens, scratch * weights[:, None]) of
                  native/native_layer_dispatch.cpp:88,129.  On the reference's
                  CUDA device, rows with the same token are bf16 atomic adds
                  (each add rounded, order unspecified); torch CPU instead sums
                  duplicate indices of one call in fp32.  So the decode group
                  (every row is token 0) is restated as one index_add_ call per
                  row in row order (one valid order of the device's adds), and a
                  group of distinct tokens as one call.

Run:  python tests/golden/make_golden.py      (writes tests/golden/*.npz)
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

HERE = Path(__file__).resolve().parent
SEED = 20261011


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def torch_route(x, gate, top_k, normalize, bias=None):
    logits = F.linear(x, gate)                                   # qwen.py:147
    scores = logits.float() if bias is None else logits.float() + bias
    probs = F.softmax(scores, dim=-1, dtype=torch.float32)      # qwen.py:148
    weights, selected = torch.sort(probs, dim=-1, descending=True, stable=True)
    weights, selected = weights[:, :top_k], selected[:, :top_k]  # qwen.py:149 + tie rule
    if normalize:
        weights = weights / weights.sum(dim=-1, keepdim=True)    # qwen.py:150-151
    return logits, selected, weights.to(x.dtype), probs          # qwen.py:152


def torch_compact_groups(selected, experts):
    n, k = selected.shape
    flat = selected.T.contiguous().view(-1)                      # runtime:25
    counts = torch.bincount(flat, minlength=experts)             # runtime:26
    order = torch.argsort(flat, stable=True)                     # runtime:28
    tokens = order.remainder(n)                                  # runtime:29
    positions = tokens * k + torch.div(order, n, rounding_mode='floor')
    return counts, tokens, positions


def torch_expert_groups(selected):
    groups = []
    for expert in sorted(set(selected.flatten().tolist())):     # qwen.py:171
        slots, tokens = torch.where((selected == expert).T)      # qwen.py:172
        groups.append((expert, tokens, slots))
    return groups


def route_case(name, T, H, E, k, normalize, *, bias=None, quantize=None, seed=SEED):
    g = torch.Generator().manual_seed(seed)
    gate = (torch.randn((E, H), generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn((T, H), generator=g).to(torch.bfloat16)
    if quantize is not None:
        # tie-heavy: few distinct gate rows and coarse activations
        gate = gate[torch.randint(0, quantize, (E,), generator=g)].contiguous()
        x = (torch.randint(-2, 3, (T, H), generator=g).float() * 0.5).to(torch.bfloat16)
    b = None if bias is None else torch.as_tensor(bias, dtype=torch.float32)
    logits, sel, w, probs = torch_route(x, gate, k, normalize, b)
    counts, tokens, positions = torch_compact_groups(sel, E)
    groups = torch_expert_groups(sel)
    g_tok = torch.cat([t for _, t, _ in groups]).numpy().astype(np.int32)
    g_pos = torch.cat([t * k + s for _, t, s in groups]).numpy().astype(np.int32)
    out = dict(x=bits(x), gate=bits(gate), logits=bits(logits), ids=sel.numpy().astype(np.int32),
               weights=bits(w), probs=probs.numpy(), counts=counts.numpy().astype(np.int32),
               perm_token=tokens.numpy().astype(np.int32), perm_pos=positions.numpy().astype(np.int32),
               groups_token=g_tok, groups_pos=g_pos,
               meta=np.array([T, H, E, k, int(normalize)], np.int64))
    if b is not None:
        out['bias'] = b.numpy()
    np.savez_compressed(HERE / f'route_{name}.npz', **out)


def expert_case(name, m, H, I, seed=SEED + 7):
    g = torch.Generator().manual_seed(seed)
    wg = (torch.randn((I, H), generator=g) * 0.02).to(torch.bfloat16)
    wu = (torch.randn((I, H), generator=g) * 0.02).to(torch.bfloat16)
    wd = (torch.randn((H, I), generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn((m, H), generator=g).to(torch.bfloat16)
    tensors = dict(gate_proj=wg, up_proj=wu, down_proj=wd)
    y = F.linear(F.silu(F.linear(x, tensors['gate_proj'])) *           # qwen.py:89-90
                 F.linear(x, tensors['up_proj']), tensors['down_proj'])
    xf = x.float()
    gate = xf @ wg.float().T                                           # qwen.py:95-98
    up = xf @ wu.float().T
    yf = ((gate * torch.sigmoid(gate)) * up) @ wd.float().T
    np.savez_compressed(HERE / f'expert_{name}.npz', x=bits(x), wg=bits(wg), wu=bits(wu), wd=bits(wd),
                        y_bf16=bits(y), y_fp32=yf.numpy())


def merge_case(name, T, H, E, k, seed=SEED + 9):
    g = torch.Generator().manual_seed(seed)
    sel = torch.argsort(torch.rand((T, E), generator=g), dim=1)[:, :k]       # k distinct experts per token
    w = torch.softmax(torch.randn((T, k), generator=g), dim=-1).to(torch.bfloat16)
    groups = torch_expert_groups(sel)                                         # (slot, token) order per expert
    parts = {e: (torch.randn((len(t), H), generator=g) * 0.5).to(torch.bfloat16) for e, t, _ in groups}
    output = torch.zeros((T, H), dtype=torch.bfloat16)                        # runtime:454 (zeros_like)
    for e, tokens, slots in groups:                                           # runtime:465 ordered=sorted(groups)
        coeff = w[tokens, slots]
        output.index_add_(0, tokens, (parts[e] * coeff[:, None]).to(output.dtype))   # runtime:466-468
    y = torch.cat([parts[e] for e, _, _ in groups])                           # grouped row order
    np.savez_compressed(HERE / f'merge_{name}.npz', ids=sel.numpy().astype(np.int32), weights=bits(w), y=bits(y),
                        out=bits(output))


def native_tail_case(name, rows, H, seed=SEED + 10):
    g = torch.Generator().manual_seed(seed)
    scratch = (torch.randn((rows, H), generator=g) * 0.5).to(torch.bfloat16)
    weights = torch.softmax(torch.randn(rows, generator=g), dim=-1).to(torch.bfloat16)
    out0 = (torch.randn((rows, H), generator=g) * 0.25).to(torch.bfloat16)
    prod = scratch * weights.unsqueeze(1)                                     # native_layer_dispatch.cpp:88
    decode = out0[:1].clone()
    for r in range(rows):                                                     # every row is token 0
        decode.index_add_(0, torch.zeros(1, dtype=torch.long), prod[r:r + 1])
    tokens = torch.randperm(rows, generator=g)                                # distinct tokens
    distinct = out0.clone()
    distinct.index_add_(0, tokens, prod)
    np.savez_compressed(HERE / f'native_tail_{name}.npz', scratch=bits(scratch), weights=bits(weights),
                        out0=bits(out0), out_decode=bits(decode), tokens=tokens.numpy(), out_distinct=bits(distinct))


def main():
    torch.set_num_threads(4)
    route_case('qwen_t64', 64, 2048, 128, 8, True)
    route_case('qwen_t1', 1, 2048, 128, 8, True, seed=SEED + 1)
    route_case('ties_t128', 128, 256, 128, 8, True, quantize=6, seed=SEED + 2)
    route_case('dsv2_t48', 48, 2048, 64, 6, False, seed=SEED + 3)
    ranks = np.arange(1, 129, dtype=np.float64)
    p = ranks ** -1.1
    p /= p.sum()
    perm = np.random.default_rng(SEED).permutation(128)
    bias = np.log(p[perm]).astype(np.float32)
    route_case('zipf_t64', 64, 2048, 128, 8, True, bias=bias, seed=SEED + 4)
    expert_case('small', 16, 256, 128)
    expert_case('h2048_m4', 4, 2048, 64)
    merge_case('t48', 48, 256, 32, 8)
    native_tail_case('r6', 6, 512)
    print('wrote', sorted(p.name for p in HERE.glob('*.npz')))


if __name__ == '__main__':
    main()
