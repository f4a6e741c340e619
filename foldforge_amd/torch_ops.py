"""The ``pytorch`` backend of the op classes: the equations in plain torch ops.

This is the engine's reference backend that FoldForge's guard falls back to for a call a
kernel backend refuses (``src/foldforge/modules/engine/policy.py:64-74`` of the
reference). It runs on whatever device its inputs are on, computes in fp32 from fp32
parameters and returns the input dtype. Equations: the reference's legacy statements
(``legacy/reference/triangle.py:39-49``, ``legacy/attention.py:108-163``,
``legacy/reference/attention.py:77-100``, ``legacy/reference/transition.py:40-41``,
``legacy/transformer.py:93-137``, ``legacy/attention.py:203-223``), under the engine's
``[B, N]`` key mask.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

Tensor = torch.Tensor

#: Replacement value of masked logits (``legacy/reference/attention.py:73``).
MASK_VALUE = -1e9


def _ln(x: Tensor, w: Tensor | None, b: Tensor | None, eps: float) -> Tensor:
    return F.layer_norm(x, x.shape[-1:], None if w is None else w.float(),
                        None if b is None else b.float(), eps)


def _lin(x: Tensor, w: Tensor, b: Tensor | None = None) -> Tensor:
    return F.linear(x, w.float(), None if b is None else b.float())


def triangle_multiplication(m, x: Tensor, mask: Tensor, *, residual: bool = True) -> Tensor:
    """``m``: a TriangleMultiplication module (parameters in engine names)."""
    dtype = x.dtype
    z = x.float()
    h = _ln(z, m.ln_pair.weight, m.ln_pair.bias, m.ln_pair.eps)
    km = mask.to(z.dtype)
    pm = (km[:, :, None] * km[:, None, :])[..., None]
    a = _lin(h, m.to_left.weight) * pm * torch.sigmoid(_lin(h, m.to_left_gate.weight))
    b = _lin(h, m.to_right.weight) * pm * torch.sigmoid(_lin(h, m.to_right_gate.weight))
    a, b = a.permute(0, 3, 1, 2), b.permute(0, 3, 1, 2)
    p = a @ b.transpose(-1, -2) if m.outgoing else a.transpose(-1, -2) @ b
    p = p.permute(0, 2, 3, 1)
    if getattr(m, "divide_by_length", False):
        count = mask.any(dim=0).sum().clamp_min(1).to(p.dtype)
        p = p / count
    y = _lin(_ln(p, m.ln_out.weight, m.ln_out.bias, m.ln_out.eps), m.to_out.weight)
    delta = y * torch.sigmoid(_lin(h, m.to_gate.weight))
    return (z + delta if residual else delta).to(dtype)


def _attend(q: Tensor, k: Tensor, v: Tensor, bias: Tensor, keep: Tensor, scale: float) -> Tensor:
    logits = (q * scale) @ k.transpose(-1, -2) + bias
    logits = logits.masked_fill(~keep, MASK_VALUE)
    return logits.softmax(dim=-1) @ v


def triangle_attention(m, x: Tensor, mask: Tensor, *, residual: bool = True,
                       row_budget: int = 1 << 28) -> Tensor:
    """``m``: a TriangleAttention module; rows are processed in chunks of bounded logits."""
    dtype = x.dtype
    z = x.float()
    batch, n = z.shape[0], z.shape[1]
    h = _ln(z, m.ln_pair.weight, m.ln_pair.bias, m.ln_pair.eps)
    bias = torch.einsum("bjkc,hc->bhjk", h, m.to_bias.weight.float())
    if not m.starting:
        h = h.transpose(1, 2)
        if m.transposed_bias:
            bias = bias.transpose(-1, -2)
    heads = m.n_head
    hd = m.to_query.weight.shape[0]
    d = hd // heads
    keep = mask.to(torch.bool)
    o = torch.empty(batch, n, n, hd, dtype=z.dtype, device=z.device)
    chunk = max(1, row_budget // max(1, n * n * heads))
    for b in range(batch):
        kb = keep[b][None, None, None, :]
        for r0 in range(0, n, chunk):
            xs = h[b, r0 : r0 + chunk]
            rows = xs.shape[0]

            def split(t: Tensor) -> Tensor:
                return t.reshape(rows, n, heads, d).permute(0, 2, 1, 3)

            att = _attend(split(_lin(xs, m.to_query.weight)), split(_lin(xs, m.to_key.weight)),
                          split(_lin(xs, m.to_value.weight)), bias[b][None], kb, d**-0.5)
            o[b, r0 : r0 + rows] = att.permute(0, 2, 1, 3).reshape(rows, n, hd)
    empty = ~keep.any(dim=-1)
    o = torch.where(empty[:, None, None, None], torch.zeros_like(o), o)
    gated = torch.sigmoid(_lin(h, m.to_gate.weight, m.to_gate.bias)) * o
    y = _lin(gated, m.to_out.weight, m.to_out.bias)
    if not m.starting and (m.dual_output or not m.untransposed_output):
        y = y.transpose(1, 2)
    if m.dual_output:
        other = _lin(gated, m.to_out_t.weight, m.to_out_t.bias)
        if not m.starting:
            other = other.transpose(1, 2)
        y = y + other.transpose(1, 2)
    return (z + y if residual else y).to(dtype)


def transition(m, x: Tensor, *, residual: bool = True) -> Tensor:
    dtype = x.dtype
    z = x.float()
    h = _ln(z, m.ln_in.weight, m.ln_in.bias, m.ln_in.eps)
    y = _lin(F.silu(_lin(h, m.expand_a.weight)) * _lin(h, m.expand_b.weight), m.squeeze.weight)
    return (z + y if residual else y).to(dtype)


def layer_norm(m, x: Tensor) -> Tensor:
    return _ln(x.float(), m.weight, m.bias, m.eps).to(x.dtype)


def attention_pair_bias(m, s: Tensor, z: Tensor, mask: Tensor, extra_bias: Tensor | None = None,
                        *, residual: bool = True) -> Tensor:
    dtype = s.dtype
    x0 = s.float()
    batch, n, cs = x0.shape
    heads = m.n_head
    d = cs // heads
    x = _ln(x0, m.ln_single.weight, m.ln_single.bias, m.ln_single.eps)

    def split(t: Tensor) -> Tensor:
        return t.reshape(batch, n, heads, d).permute(0, 2, 1, 3)

    q = split(_lin(x, m.to_query.weight, m.to_query.bias))
    k = split(_lin(x, m.to_key.weight))
    v = split(_lin(x, m.to_value.weight))
    zb = _ln(z.float(), m.ln_pair.weight, None, m.ln_pair.eps)
    bias = torch.einsum("bijc,hc->bhij", zb, m.to_bias.weight.float())
    if extra_bias is not None:
        bias = bias + extra_bias.float()
    keep = mask.to(torch.bool)[:, None, None, :]
    o = _attend(q, k, v, bias, keep, d**-0.5).permute(0, 2, 1, 3).reshape(batch, n, cs)
    o = torch.where((~mask.to(torch.bool).any(dim=-1))[:, None, None], torch.zeros_like(o), o)
    gate = torch.sigmoid(_lin(x, m.to_gate.weight) + m.gate_bias)
    y = _lin(gate * o, m.to_out.weight)
    return (x0 + y if residual else y).to(dtype)


def msa_pair_weighted_averaging(m_, msa: Tensor, z: Tensor, mask: Tensor, *,
                                residual: bool = True) -> Tensor:
    """``m_``: an MSAPairWeightedAveraging module; ``msa [B, S, N, c_m]``, ``z [B, N, N, c_z]``,
    key mask ``[B, N]`` (``legacy/attention.py:203-223``)."""
    dtype = msa.dtype
    m = msa.float()
    batch, depth, n, _ = m.shape
    heads = m_.n_head
    x = _ln(m, m_.ln_msa.weight, m_.ln_msa.bias, m_.ln_msa.eps)
    zn = _ln(z.float(), m_.ln_pair.weight, None, m_.ln_pair.eps)
    logits = torch.einsum("bijc,hc->bhij", zn, m_.to_bias.weight.float())
    keep = mask.to(torch.bool)
    w = logits.masked_fill(~keep[:, None, None, :], MASK_VALUE).softmax(dim=-1)
    v = _lin(x, m_.to_value.weight).reshape(batch, depth, n, heads, -1)
    o = torch.einsum("bhij,bsjhc->bsihc", w, v).reshape(batch, depth, n, -1)
    o = torch.where((~keep.any(dim=-1))[:, None, None, None], torch.zeros_like(o), o)
    y = _lin(torch.sigmoid(_lin(x, m_.to_gate.weight)) * o, m_.to_out.weight)
    return (m + y if residual else y).to(dtype)


def outer_product_mean(m_, msa: Tensor, mask: Tensor, *, residual: Tensor | None = None) -> Tensor:
    """``m_``: an OuterProductMean module; ``msa [B, S, N, c_m]``, row mask ``[B, S, N]``
    (``legacy/primitives.py:80-136``, ``legacy/reference/attention.py:57-74``)."""
    dtype = msa.dtype
    batch, depth, n, _ = msa.shape
    x = _ln(msa.float(), m_.ln_msa.weight, m_.ln_msa.bias, m_.ln_msa.eps)
    keep = mask.to(torch.float32)
    left = _lin(x, m_.to_left.weight, m_.to_left.bias) * keep[..., None]
    right = _lin(x, m_.to_right.weight, m_.to_right.bias) * keep[..., None]
    if m_.groups == 1:
        o = torch.einsum("bsic,bsje->bijce", left, right).reshape(batch, n, n, -1)
        count = torch.einsum("bsi,bsj->bij", keep, keep)[..., None]
        d = count.clamp_min(1.0) if m_.count_offset is None else count + m_.count_offset
        if m_.normalize_before_proj:
            y = _lin(o / d, m_.to_out.weight, m_.to_out.bias)
        else:
            y = _lin(o, m_.to_out.weight, m_.to_out.bias) / d
    else:
        g = m_.groups
        o = torch.einsum("bsigc,bsjge->bijgce", left.unflatten(-1, (g, -1)),
                         right.unflatten(-1, (g, -1))).reshape(batch, n, n, -1)
        pn = m_.product_norm
        y = _lin(_ln(o, pn.weight, pn.bias, pn.eps), m_.to_out.weight, m_.to_out.bias)
    if residual is not None:
        y = residual.float() + y
    return y.to(dtype)
