"""Pure-Python fp64 loop restatements of the pair-stack ops for tiny shapes (test oracle).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``). Written element by element
from the equations (no matrix products, no einsum) so that they pin
``oracle.pairstack`` independently: a dropped term, a swapped index or a
transposed operand in either shows up as a mismatch. Inputs are nested-index
numpy fp64 arrays; every loop is explicit. Sizes must stay tiny (N <= 8).

Equations (reference paths as in ``oracle/pairstack.py``):
``legacy/reference/triangle.py:39-49``, ``legacy/attention.py:108-163``,
``legacy/reference/attention.py:96-101``, ``legacy/reference/transition.py:40-41``,
``legacy/transformer.py:93-137``, ``legacy/attention.py:203-223`` (MSA pair-weighted
averaging), ``legacy/primitives.py:80-156`` (outer product mean).
"""

from __future__ import annotations

import math

import numpy as np

MASK_VALUE = -1e9


def _sigmoid(x: float) -> float:
    return 1.0 / (1.0 + math.exp(-x))


def _silu(x: float) -> float:
    return x * _sigmoid(x)


def layer_norm_vec(x, w, b, eps: float) -> list[float]:
    n = len(x)
    mean = sum(x) / n
    var = sum((v - mean) ** 2 for v in x) / n
    inv = 1.0 / math.sqrt(var + eps)
    return [
        (x[i] - mean) * inv * (1.0 if w is None else w[i]) + (0.0 if b is None else b[i])
        for i in range(n)
    ]


def _matvec(w, x) -> list[float]:
    """``y[o] = sum_i w[o][i] x[i]``."""
    return [sum(w[o][i] * x[i] for i in range(len(x))) for o in range(len(w))]


def _softmax_row(logits: list[float]) -> list[float]:
    mx = max(logits)
    e = [math.exp(v - mx) for v in logits]
    s = sum(e)
    return [v / s for v in e]


def triangle_multiplication(z, mask, p, *, outgoing: bool, length_divided: bool = False,
                            eps: float = 1e-5):
    """``z [B, N, N, c]`` fp64, ``mask [B, N]``; ``p`` numpy fp64 params (engine names).
    ``length_divided``: every contraction sum divided by the count of columns j with a real
    token in some batch element (at least 1)."""
    batch, n, _, c = z.shape
    hid = p["to_left.weight"].shape[0]
    out = np.array(z, dtype=np.float64, copy=True)
    length = 0
    for j in range(n):
        if any(bool(mask[b, j]) for b in range(batch)):
            length += 1
    divisor = float(max(length, 1)) if length_divided else 1.0
    for b in range(batch):
        xh = [[layer_norm_vec(z[b, i, j], p["ln_pair.weight"], p["ln_pair.bias"], eps)
               for j in range(n)] for i in range(n)]
        a = [[[0.0] * hid for _ in range(n)] for _ in range(n)]
        bb = [[[0.0] * hid for _ in range(n)] for _ in range(n)]
        for i in range(n):
            for k in range(n):
                m = float(mask[b, i]) * float(mask[b, k])
                left = _matvec(p["to_left.weight"], xh[i][k])
                lg = _matvec(p["to_left_gate.weight"], xh[i][k])
                right = _matvec(p["to_right.weight"], xh[i][k])
                rg = _matvec(p["to_right_gate.weight"], xh[i][k])
                for h in range(hid):
                    a[i][k][h] = left[h] * m * _sigmoid(lg[h])
                    bb[i][k][h] = right[h] * m * _sigmoid(rg[h])
        for i in range(n):
            for j in range(n):
                pv = [0.0] * hid
                for h in range(hid):
                    acc = 0.0
                    for k in range(n):
                        if outgoing:
                            acc += a[i][k][h] * bb[j][k][h]
                        else:
                            acc += a[k][i][h] * bb[k][j][h]
                    pv[h] = acc / divisor
                y = _matvec(p["to_out.weight"],
                            layer_norm_vec(pv, p["ln_out.weight"], p["ln_out.bias"], eps))
                g = _matvec(p["to_gate.weight"], xh[i][j])
                for ch in range(c):
                    out[b, i, j, ch] = z[b, i, j, ch] + y[ch] * _sigmoid(g[ch])
    return out


def triangle_attention(z, mask, p, *, starting: bool, n_head: int,
                       transposed_bias: bool = False, untransposed_output: bool = False,
                       dual_output: bool = False, eps: float = 1e-5):
    """Row (starting) or column (ending) attention with the shared pair bias, fp64 loops.
    Gate / output biases where ``p`` holds them; ``untransposed_output``: the ending node's
    update lands at (row, query), not (query, row); ``dual_output``: ``to_out_t`` of the same
    gated values lands at the mirror of the update's position."""
    batch, n, _, c = z.shape
    hd = p["to_query.weight"].shape[0]
    d = hd // n_head
    scale = 1.0 / math.sqrt(d)
    out = np.array(z, dtype=np.float64, copy=True)
    for b in range(batch):
        xh = [[layer_norm_vec(z[b, i, j], p["ln_pair.weight"], p["ln_pair.bias"], eps)
               for j in range(n)] for i in range(n)]
        bias = [[[0.0] * n for _ in range(n)] for _ in range(n_head)]
        for h in range(n_head):
            for j in range(n):
                for k in range(n):
                    src = xh[k][j] if (not starting and transposed_bias) else xh[j][k]
                    bias[h][j][k] = sum(p["to_bias.weight"][h][ch] * src[ch] for ch in range(c))
        any_key = any(bool(mask[b, k]) for k in range(n))
        for r in range(n):
            # the sequence of the row: x[r, s] (starting) or x[s, r] (ending)
            seq = [xh[r][s] if starting else xh[s][r] for s in range(n)]
            q = [_matvec(p["to_query.weight"], v) for v in seq]
            kk = [_matvec(p["to_key.weight"], v) for v in seq]
            vv = [_matvec(p["to_value.weight"], v) for v in seq]
            gg = [_matvec(p["to_gate.weight"], v) for v in seq]
            for j in range(n):
                o = [0.0] * hd
                for h in range(n_head):
                    logits = []
                    for k in range(n):
                        dot = sum(q[j][h * d + e] * kk[k][h * d + e] for e in range(d))
                        val = dot * scale + bias[h][j][k]
                        logits.append(val if bool(mask[b, k]) else MASK_VALUE)
                    w = _softmax_row(logits)
                    for e in range(d):
                        o[h * d + e] = sum(w[k] * vv[k][h * d + e] for k in range(n)) if any_key else 0.0
                gb = p.get("to_gate.bias")
                gated = [_sigmoid(gg[j][f] + (gb[f] if gb is not None else 0.0)) * o[f]
                         for f in range(hd)]
                y = _matvec(p["to_out.weight"], gated)
                if p.get("to_out.bias") is not None:
                    y = [y[ch] + p["to_out.bias"][ch] for ch in range(c)]
                zi, zj = (r, j) if starting or (untransposed_output and not dual_output) else (j, r)
                for ch in range(c):
                    out[b, zi, zj, ch] += y[ch]
                if dual_output:
                    yt = _matvec(p["to_out_t.weight"], gated)
                    for ch in range(c):
                        out[b, zj, zi, ch] += yt[ch] + (p["to_out_t.bias"][ch] if p.get("to_out_t.bias") is not None else 0.0)
    return out


def transition(x, p, *, eps: float = 1e-5):
    """``x [..., c]`` fp64: ``x + squeeze(silu(expand_a h) * expand_b h)``."""
    flat = np.asarray(x, dtype=np.float64).reshape(-1, x.shape[-1])
    out = flat.copy()
    for r in range(flat.shape[0]):
        h = layer_norm_vec(flat[r], p["ln_in.weight"], p["ln_in.bias"], eps)
        a = _matvec(p["expand_a.weight"], h)
        bv = _matvec(p["expand_b.weight"], h)
        hid = [_silu(a[i]) * bv[i] for i in range(len(a))]
        y = _matvec(p["squeeze.weight"], hid)
        for ch in range(flat.shape[1]):
            out[r, ch] += y[ch]
    return out.reshape(x.shape)


def attention_pair_bias(s, z, mask, p, *, n_head: int, gate_bias: float = 0.0,
                        extra_bias=None, eps: float = 1e-5):
    """Single-track attention with the pair bias, fp64 loops; ``extra_bias [B, H, N, N]`` is
    added to every logit where given."""
    batch, n, cs = s.shape
    d = cs // n_head
    scale = 1.0 / math.sqrt(d)
    out = np.array(s, dtype=np.float64, copy=True)
    for b in range(batch):
        x = [layer_norm_vec(s[b, i], p["ln_single.weight"], p["ln_single.bias"], eps)
             for i in range(n)]
        q = [[v + bq for v, bq in zip(_matvec(p["to_query.weight"], xi), p["to_query.bias"])]
             for xi in x]
        kk = [_matvec(p["to_key.weight"], xi) for xi in x]
        vv = [_matvec(p["to_value.weight"], xi) for xi in x]
        gg = [_matvec(p["to_gate.weight"], xi) for xi in x]
        zb = [[_matvec(p["to_bias.weight"], layer_norm_vec(z[b, i, j], p["ln_pair.weight"], None, eps))
               for j in range(n)] for i in range(n)]
        any_key = any(bool(mask[b, k]) for k in range(n))
        for i in range(n):
            o = [0.0] * cs
            for h in range(n_head):
                logits = []
                for k in range(n):
                    dot = sum(q[i][h * d + e] * kk[k][h * d + e] for e in range(d))
                    val = dot * scale + zb[i][k][h]
                    if extra_bias is not None:
                        val += float(extra_bias[b, h, i, k])
                    logits.append(val if bool(mask[b, k]) else MASK_VALUE)
                w = _softmax_row(logits)
                for e in range(d):
                    o[h * d + e] = sum(w[k] * vv[k][h * d + e] for k in range(n)) if any_key else 0.0
            gated = [_sigmoid(gg[i][f] + gate_bias) * o[f] for f in range(cs)]
            y = _matvec(p["to_out.weight"], gated)
            for ch in range(cs):
                out[b, i, ch] += y[ch]
    return out


def msa_pair_weighted_averaging(m, z, mask, p, *, n_head: int, eps: float = 1e-5):
    """MSA pair-weighted averaging, fp64 loops: one softmax over keys j per (head, query i),
    shared by every MSA row s."""
    batch, depth, n, cm = m.shape
    hd = len(p["to_value.weight"])
    d = hd // n_head
    out = np.array(m, dtype=np.float64, copy=True)
    for b in range(batch):
        any_key = any(bool(mask[b, k]) for k in range(n))
        w = [[None] * n for _ in range(n_head)]
        for i in range(n):
            zb = [_matvec(p["to_bias.weight"], layer_norm_vec(z[b, i, j], p["ln_pair.weight"], None, eps))
                  for j in range(n)]
            for h in range(n_head):
                w[h][i] = _softmax_row([zb[j][h] if bool(mask[b, j]) else MASK_VALUE for j in range(n)])
        for s in range(depth):
            x = [layer_norm_vec(m[b, s, j], p["ln_msa.weight"], p["ln_msa.bias"], eps) for j in range(n)]
            v = [_matvec(p["to_value.weight"], xj) for xj in x]
            for i in range(n):
                g = _matvec(p["to_gate.weight"], x[i])
                o = [0.0] * hd
                for h in range(n_head):
                    for c in range(d):
                        f = h * d + c
                        o[f] = sum(w[h][i][j] * v[j][f] for j in range(n)) if any_key else 0.0
                gated = [_sigmoid(g[f]) * o[f] for f in range(hd)]
                y = _matvec(p["to_out.weight"], gated)
                for ch in range(cm):
                    out[b, s, i, ch] += y[ch]
    return out


def outer_product_mean(m, rows_mask, p, *, count_offset=1e-3, normalize_before_proj=False,
                       groups: int = 1, eps: float = 1e-5, product_norm_eps: float = 0.1):
    """Outer product mean (raw update), fp64 loops. ``to_out.weight`` column ``g K K + c K + e``
    multiplies the product of left channel ``g K + c`` and right channel ``g K + e``."""
    batch, depth, n, _ = m.shape
    hidden = len(p["to_left.weight"])
    k = hidden // groups
    cz = len(p["to_out.weight"])
    bl, br = p.get("to_left.bias"), p.get("to_right.bias")
    out = np.zeros((batch, n, n, cz))
    for b in range(batch):
        left = [[None] * n for _ in range(depth)]
        right = [[None] * n for _ in range(depth)]
        for s in range(depth):
            for i in range(n):
                x = layer_norm_vec(m[b, s, i], p["ln_msa.weight"], p["ln_msa.bias"], eps)
                keep = 1.0 if bool(rows_mask[b, s, i]) else 0.0
                lv = _matvec(p["to_left.weight"], x)
                rv = _matvec(p["to_right.weight"], x)
                left[s][i] = [keep * (lv[c] + (bl[c] if bl is not None else 0.0)) for c in range(hidden)]
                right[s][i] = [keep * (rv[c] + (br[c] if br is not None else 0.0)) for c in range(hidden)]
        for i in range(n):
            for j in range(n):
                o = [0.0] * (groups * k * k)
                for g in range(groups):
                    for c in range(k):
                        for e in range(k):
                            o[g * k * k + c * k + e] = sum(left[s][i][g * k + c] * right[s][j][g * k + e]
                                                           for s in range(depth))
                if groups > 1:
                    o = layer_norm_vec(o, p["product_norm.weight"], p["product_norm.bias"], product_norm_eps)
                    y = _matvec(p["to_out.weight"], o)
                    for f in range(cz):
                        out[b, i, j, f] = y[f] + p["to_out.bias"][f]
                    continue
                cnt = sum((1.0 if bool(rows_mask[b, s, i]) else 0.0) * (1.0 if bool(rows_mask[b, s, j]) else 0.0)
                          for s in range(depth))
                d = max(cnt, 1.0) if count_offset is None else cnt + count_offset
                if normalize_before_proj:
                    y = _matvec(p["to_out.weight"], [v / d for v in o])
                    for f in range(cz):
                        out[b, i, j, f] = y[f] + p["to_out.bias"][f]
                else:
                    y = _matvec(p["to_out.weight"], o)
                    for f in range(cz):
                        out[b, i, j, f] = (y[f] + p["to_out.bias"][f]) / d
    return out
