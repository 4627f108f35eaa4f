"""The reference projection-engine step as torch CPU library calls (test infrastructure only).

This is the CPU baseline bench.py times beside the GPU number, and nothing else: only tests/,
``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg may use it.  It restates the op
sequence of STACRFunction.forward/backward (stacr/layers.py:113-199) with the helpers it calls,
so the time it takes is what the reference's own path costs on the same cores:

  save      coeff = act @ q in the activation dtype (:135-137); per chunk of rows the residual
            act - coeff @ q^T (:32, :73) and torch.topk of its magnitudes, with the chunk_topk
            budget trim (:16-41) or the global_topk running merge (:69-80);
            quantize_values: fp32 per-tensor scale, round half to even, clamp (stacr/quant.py:49-65)
  backward  (G^T coeff) q^T in G's dtype (:172-173); the dequantized entries as a coalesced
            COO matrix and torch.sparse.mm against G in fp32 (:174-193); transpose for Conv1D and
            cast to the weight dtype (:194-196)
"""
from __future__ import annotations

import torch


def _budget_count(budget: float, n: int) -> int:
    return int(round(float(budget) * n))  # Python's half-to-even round, as stacr/layers.py:25,33,51


def _chunk_residuals(act, coeff, q, chunk_rows):
    """(first flat offset, flat residual) of each chunk of rows (stacr/layers.py:30-32, 70-73)."""
    rows, feats = act.shape
    for start in range(0, rows, max(1, int(chunk_rows))):
        stop = min(start + int(chunk_rows), rows)
        yield start * feats, (act[start:stop] - coeff[start:stop].mm(q.t())).reshape(-1)


def select(act, coeff, q, mode: str, budget: float, chunk_rows: int):
    """(flat indices, values) of chunk_topk / global_topk on the CPU (stacr/layers.py:16-41, 69-80)."""
    total = act.numel()
    k_total = _budget_count(budget, total)
    if k_total <= 0:
        return None, None
    if mode == "global_topk":
        kept_i = kept_v = None
        for offset, flat in _chunk_residuals(act, coeff, q, chunk_rows):
            pick = torch.topk(flat.abs(), min(k_total, flat.numel()), sorted=False).indices
            cand_i, cand_v = pick + offset, flat[pick]
            if kept_i is not None:
                cand_i, cand_v = torch.cat((kept_i, cand_i)), torch.cat((kept_v, cand_v))
            best = torch.topk(cand_v.abs(), min(k_total, cand_v.numel()), sorted=False).indices
            kept_i, kept_v = cand_i[best], cand_v[best]
        idx, val = kept_i, kept_v
    else:
        parts_i, parts_v = [], []
        for offset, flat in _chunk_residuals(act, coeff, q, chunk_rows):
            k = max(1, min(flat.numel(), _budget_count(budget, flat.numel())))
            pick = torch.topk(flat.abs(), k, sorted=False).indices
            parts_i.append(pick + offset)
            parts_v.append(flat[pick])
        idx, val = torch.cat(parts_i), torch.cat(parts_v)
        if idx.numel() > k_total:
            best = torch.topk(val.abs(), k_total, sorted=False).indices
            idx, val = idx[best], val[best]
    return idx.to(torch.int32 if total < 2**31 - 1 else torch.int64), val


def quantize(values, bits: int):
    """(codes, fp32 scale) of quantize_values for bits 8 / 4 before nibble packing (stacr/quant.py:49-65)."""
    qmax = 127 if bits == 8 else 7
    v = values.float()
    scale = (v.abs().max() / qmax).clamp_min(torch.finfo(torch.float32).tiny)
    return torch.round(v / scale).clamp(-qmax - 1, qmax).to(torch.int8), scale


def save(act, q, mode: str, budget: float, chunk_rows: int, bits: int):
    """coeff, idx, codes, scale of one forward's save (stacr/layers.py:135-148)."""
    coeff = act.mm(q)
    idx, val = select(act, coeff, q, mode, budget, chunk_rows)
    if idx is None:
        return coeff, None, None, None
    codes, scale = quantize(val, bits)
    return coeff, idx, codes, scale


def weight_grad(g, coeff, q, idx, codes, scale, in_features: int, transposed: bool, weight_dtype):
    """dW from the saved factors (stacr/layers.py:172-196)."""
    grad = g.t().mm(coeff.to(g.dtype)).mm(q.to(g.dtype).t())
    if idx is not None and idx.numel():
        values = codes.float() * scale
        flat = idx.long()
        coords = torch.stack((torch.div(flat, in_features, rounding_mode="floor"), flat % in_features))
        sparse = torch.sparse_coo_tensor(coords, values, size=(g.shape[0], in_features)).coalesce()
        grad = grad + torch.sparse.mm(sparse.t(), g.float()).t().to(grad.dtype)
    if transposed:
        grad = grad.t()
    return grad.to(weight_dtype)


def layer_step(act, q, g, *, mode: str, budget: float, chunk_rows: int, bits: int, transposed: bool,
               weight_dtype):
    """One save + weight gradient of the reference path on CPU tensors."""
    coeff, idx, codes, scale = save(act, q, mode, budget, chunk_rows, bits)
    return weight_grad(g, coeff, q, idx, codes, scale, act.shape[1], transposed, weight_dtype)
