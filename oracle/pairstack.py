"""fp32 / fp64 CPU restatement of the Pairformer pair-stack equations (test oracle).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): imported by ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg, never by the
``foldforge_amd`` package.

Every function takes the engine's parameter names (the ``state_dict`` keys of one
op module, e.g. ``"to_left.weight"``) and batched engine-layout inputs:
pair ``z [B, N, N, c]``, key mask ``mask [B, N]`` (bool), single ``s [B, N, c_s]``.
Each returns ``x + f(x)`` (the engine ops own their residual) in ``dtype``.

Reference equations followed (paths relative to the reference tree):

* LayerNorm: ``torch.nn.LayerNorm`` as used by
  ``src/foldforge/models/checkpoints/legacy/attention.py:90`` and
  ``legacy/triangle_multiplication.py:40,43``; fp32 affine
  (``src/foldforge/modules/engine/modules.py:230-238``).
* Triangle multiplication: ``legacy/reference/triangle.py:19-49`` (mask multiply
  before the sigmoid gate, ``:40-43``; equations ``:45``), bound by
  ``legacy/routing.py:82-102`` and the engine split of
  ``legacy/released.py:135-173`` (the engine's incoming contracts
  ``left[k, i] * right[k, j]``, ``released.py:143-145``).
* Triangle attention: ``legacy/attention.py:108-163`` with
  ``legacy/reference/attention.py:77-100`` (bias added before the -1e9
  replacement mask, ``:96-101``); bias from the un-transposed pair for AF3
  (``attention.py:144-147``), transposed for the OpenFold lineage
  (``src/foldforge/modules/dense/spec.py:116-125``); output turned back
  (``attention.py:161-162``). Row chunking as ``attention.py:23-57``.
* Transition: ``legacy/reference/transition.py:40-41`` with
  ``src/foldforge/modules/dense/diffusion_transformer.py:36-44`` (SwiGLU, packed
  ``transition1`` split by ``chunk(2)`` into ``expand_a`` / ``expand_b``,
  ``legacy/released.py:211-224``).
* Attention with pair bias: ``legacy/transformer.py:93-137`` and
  ``legacy/pairformer.py:204-229`` (engine names ``legacy/released.py:281-315``;
  the pair norm's offset is dropped, ``released.py:268-270``).
* Block: the sequential AF3 order of ``legacy/pairformer.py:191-230``.
* MSA pair-weighted averaging: ``legacy/attention.py:174-229`` (``MSAAttention``; engine
  names ``legacy/released.py:253-278``, the pair norm's offset dropped), called with the
  engine's column key mask ``[B, N]`` (``src/foldforge/modules/engine/graph.py:295-305``).
* Outer product mean: ``legacy/primitives.py:80-156`` and
  ``legacy/reference/attention.py:57-74`` (AF3's released contraction and divisor), with the
  engine's forms (``src/foldforge/modules/engine/modules.py:184-210``) and names
  (``legacy/released.py:227-251``); returns the raw update.

The engine takes a ``[B, N]`` key mask (``src/foldforge/modules/engine/graph.py:214-218``)
where the legacy graph takes the outer-product pair mask; the two agree on valid
pairs, which is all the reference tests compare
(``tests/kernels/test_released_conversions.py:61-64``). Here padded query rows are
computed like valid rows under the key mask, and a batch element without any
valid key gets a zero attention output (the legacy graph would average
uniformly over the -1e9 logits; no valid pair is affected either way).
"""

from __future__ import annotations

from collections.abc import Mapping

import torch
import torch.nn.functional as F

Tensor = torch.Tensor
Params = Mapping[str, Tensor]

#: The replacement value of masked logits (``legacy/reference/attention.py:73``).
MASK_VALUE = -1e9


def _p(params: Params, name: str, dtype: torch.dtype) -> Tensor:
    return params[name].detach().to("cpu", dtype)


def layer_norm(
    x: Tensor, weight: Tensor | None, bias: Tensor | None, eps: float = 1e-5
) -> Tensor:
    """``(x - mean) / sqrt(var + eps) * weight + bias`` over the last axis (biased variance)."""
    mean = x.mean(dim=-1, keepdim=True)
    var = (x - mean).square().mean(dim=-1, keepdim=True)
    y = (x - mean) / torch.sqrt(var + eps)
    if weight is not None:
        y = y * weight
    if bias is not None:
        y = y + bias
    return y


def layer_norm_linear(
    x: Tensor, ln_w: Tensor | None, ln_b: Tensor | None, weight: Tensor, bias: Tensor | None = None,
    *, activation: str = "none", eps: float = 1e-5, dtype: torch.dtype = torch.float32,
) -> Tensor:
    """``act(LN(x) W^T + b)``: the LayerNorm-fed projection every pair op starts with
    (``legacy/reference/triangle.py:39-43``, ``legacy/attention.py:111-124``), as one function
    (the engine's ``layer_norm_linear``, ``docs/guides/ENGINE-2.4.2.md:21``)."""
    h = layer_norm(x.to(dtype), None if ln_w is None else ln_w.to(dtype),
                   None if ln_b is None else ln_b.to(dtype), eps)
    y = h @ weight.to(dtype).T
    if bias is not None:
        y = y + bias.to(dtype)
    if activation == "sigmoid":
        return torch.sigmoid(y)
    if activation == "silu":
        return y * torch.sigmoid(y)
    if activation == "relu":
        return y.clamp_min(0)
    if activation != "none":
        raise ValueError(f"unknown activation {activation!r}")
    return y


def swiglu_ffn(x: Tensor, w_a: Tensor, w_b: Tensor, w_out: Tensor, residual: Tensor | None = None,
               *, dtype: torch.dtype = torch.float32) -> Tensor:
    """``(silu(x W_a^T) * (x W_b^T)) W_out^T`` (+ ``residual``): the transition's body without its
    LayerNorm (``legacy/reference/transition.py:40-41``; the engine's ``swiglu_ffn``,
    ``docs/guides/ENGINE-2.4.2.md:18``)."""
    h = x.to(dtype)
    a = h @ w_a.to(dtype).T
    y = (a * torch.sigmoid(a) * (h @ w_b.to(dtype).T)) @ w_out.to(dtype).T
    return y if residual is None else residual.to(dtype) + y


def _pair_mask(mask: Tensor, dtype: torch.dtype) -> Tensor:
    m = mask.to("cpu", dtype)
    return m[:, :, None] * m[:, None, :]


def triangle_multiplication(
    z: Tensor,
    mask: Tensor,
    params: Params,
    *,
    outgoing: bool,
    length_divided: bool = False,
    eps: float = 1e-5,
    dtype: torch.dtype = torch.float32,
) -> Tensor:
    """``z + (LN_out(P) W_out^T) * sigmoid(x W_g^T)``, ``x = LN_pair(z)``.

    ``A = (x W_l^T) * M * sigmoid(x W_lg^T)``, ``B`` likewise with the right
    weights, ``M[i, k] = mask_i mask_k``; outgoing ``P[i, j] = sum_k A[i, k] B[j, k]``,
    incoming ``P[i, j] = sum_k A[k, i] B[k, j]``
    (``legacy/reference/triangle.py:39-49``, ``legacy/released.py:143-145``).
    ``length_divided`` (RoseTTAFold3's exact form): ``P`` divided by the real length ``L``
    before the centre norm, ``L`` the number of positions real in any batch element, at
    least 1 (``legacy/routing.py:33-55``, ``legacy/reference/triangle.py:46-48``).
    """
    z = z.detach().to("cpu", dtype)
    x = layer_norm(
        z, _p(params, "ln_pair.weight", dtype), _p(params, "ln_pair.bias", dtype), eps
    )
    pm = _pair_mask(mask, dtype)[..., None]
    a = (x @ _p(params, "to_left.weight", dtype).T) * pm
    a = a * torch.sigmoid(x @ _p(params, "to_left_gate.weight", dtype).T)
    b = (x @ _p(params, "to_right.weight", dtype).T) * pm
    b = b * torch.sigmoid(x @ _p(params, "to_right_gate.weight", dtype).T)
    # channel-major batched products: [B, h, N, N]
    a, b = a.permute(0, 3, 1, 2), b.permute(0, 3, 1, 2)
    if outgoing:
        p = a @ b.transpose(-1, -2)
    else:
        p = a.transpose(-1, -2) @ b
    p = p.permute(0, 2, 3, 1)
    if length_divided:
        p = p / max(1, int(mask.to("cpu").bool().any(dim=0).sum()))
    y = layer_norm(
        p, _p(params, "ln_out.weight", dtype), _p(params, "ln_out.bias", dtype), eps
    )
    y = y @ _p(params, "to_out.weight", dtype).T
    g = torch.sigmoid(x @ _p(params, "to_gate.weight", dtype).T)
    return z + y * g


def _masked_softmax_attention(
    q: Tensor, k: Tensor, v: Tensor, bias: Tensor, key_mask: Tensor, scale: float
) -> Tensor:
    """``softmax(q k^T * scale + bias, masked keys replaced by -1e9) v`` on ``[..., H, L, D]``.

    ``key_mask`` broadcasts to ``[..., 1, 1, L]`` (True = keep); the replacement comes
    after the bias (``legacy/reference/attention.py:96-101``).
    """
    logits = (q * scale) @ k.transpose(-1, -2) + bias
    logits = logits.masked_fill(~key_mask, MASK_VALUE)
    return logits.softmax(dim=-1) @ v


def triangle_attention(
    z: Tensor,
    mask: Tensor,
    params: Params,
    *,
    starting: bool,
    n_head: int,
    transposed_bias: bool = False,
    untransposed_output: bool = False,
    dual_output: bool = False,
    eps: float = 1e-5,
    dtype: torch.dtype = torch.float32,
    row_chunk: int | None = None,
) -> Tensor:
    """Triangle attention around the starting (rows) or ending (columns) node.

    ``x = LN_pair(z)``; ``bias[h, j, k] = x[j, k] . W_b[h]`` from the un-transposed
    ``x`` (AF3) or its transpose (``transposed_bias``, the ending node of the
    OpenFold lineage); for every row ``r`` of ``x`` (of ``x^T`` when ending):
    ``o[r, j] = softmax_k(q[r, j] . k[r, k] / sqrt(D) + bias[h, j, k]) v[r, k]``;
    ``y = (sigmoid(x W_g^T + b_g) * o) W_out^T + b_out`` (the biases where ``params`` holds
    them: RoseTTAFold3, ``legacy/attention.py:97-102``), turned back when ending
    (``legacy/attention.py:108-163``). ``untransposed_output`` (Chai-1's trunk): the ending
    node's ``y`` is added as it stands, not turned back (``attention.py:84-88,160-163``).
    ``dual_output`` (Chai-1's confidence head): a second projection ``to_out_t`` of the same
    gated ``o``, turned back like ``y`` and then transposed over the pair axes, is added too
    (``attention.py:129-131,152-158``).
    """
    z = z.detach().to("cpu", dtype)
    batch, n = z.shape[0], z.shape[1]
    x = layer_norm(
        z, _p(params, "ln_pair.weight", dtype), _p(params, "ln_pair.bias", dtype), eps
    )
    bias = torch.einsum("bjkc,hc->bhjk", x, _p(params, "to_bias.weight", dtype))
    if not starting:
        x = x.transpose(1, 2)
        if transposed_bias:
            bias = bias.transpose(-1, -2)
    wq, wk, wv = (
        _p(params, f"to_{name}.weight", dtype) for name in ("query", "key", "value")
    )
    hd = wq.shape[0]
    d = hd // n_head
    scale = d**-0.5
    key_mask = mask.to("cpu", torch.bool)
    out = torch.empty(batch, n, n, hd, dtype=dtype)
    chunk = row_chunk or max(1, (1 << 26) // max(1, n * n * n_head))
    for b in range(batch):
        keep = key_mask[b][None, None, None, :]
        for r0 in range(0, n, chunk):
            xs = x[b, r0 : r0 + chunk]  # [R, S, c]
            rows = xs.shape[0]

            def heads(t: Tensor) -> Tensor:
                return t.reshape(rows, n, n_head, d).permute(0, 2, 1, 3)

            q, k, v = heads(xs @ wq.T), heads(xs @ wk.T), heads(xs @ wv.T)
            o = _masked_softmax_attention(q, k, v, bias[b][None], keep, scale)
            o = o.permute(0, 2, 1, 3).reshape(rows, n, hd)
            if not bool(key_mask[b].any()):
                o = torch.zeros_like(o)
            out[b, r0 : r0 + rows] = o
    def linear(v: Tensor, name: str) -> Tensor:
        y = v @ _p(params, f"{name}.weight", dtype).T
        return y + _p(params, f"{name}.bias", dtype) if f"{name}.bias" in params else y

    gated = torch.sigmoid(linear(x, "to_gate")) * out
    y = linear(gated, "to_out")
    if not starting and (dual_output or not untransposed_output):
        y = y.transpose(1, 2)
    if dual_output:
        other = linear(gated, "to_out_t")
        if not starting:
            other = other.transpose(1, 2)
        y = y + other.transpose(1, 2)
    return z + y


def transition(
    x: Tensor, params: Params, *, eps: float = 1e-5, dtype: torch.dtype = torch.float32
) -> Tensor:
    """``x + (silu(h W_a^T) * (h W_b^T)) W_s^T``, ``h = LN_in(x)`` (``legacy/reference/transition.py:40-41``)."""
    x = x.detach().to("cpu", dtype)
    h = layer_norm(
        x, _p(params, "ln_in.weight", dtype), _p(params, "ln_in.bias", dtype), eps
    )
    a = h @ _p(params, "expand_a.weight", dtype).T
    b = h @ _p(params, "expand_b.weight", dtype).T
    return x + (F.silu(a) * b) @ _p(params, "squeeze.weight", dtype).T


def attention_pair_bias(
    s: Tensor,
    z: Tensor,
    mask: Tensor,
    params: Params,
    *,
    n_head: int,
    gate_bias: float = 0.0,
    extra_bias: Tensor | None = None,
    eps: float = 1e-5,
    dtype: torch.dtype = torch.float32,
) -> Tensor:
    """Single-track attention with pair bias (``legacy/transformer.py:93-137``).

    ``x = LN_single(s)``; ``q = x W_q^T + b_q``, ``k = x W_k^T``, ``v = x W_v^T``;
    ``bias[h, i, j] = LN_pair(z)[i, j] . W_b[h]`` (norm without offset), plus
    ``extra_bias`` (broadcast to ``[B, H, N, N]``: OpenDDE's structural bias,
    ``legacy/pairformer.py:216-218``) where given;
    ``s + (sigmoid(x W_g^T + gate_bias) * attn) W_out^T``.
    """
    s = s.detach().to("cpu", dtype)
    z = z.detach().to("cpu", dtype)
    batch, n, cs = s.shape
    x = layer_norm(
        s, _p(params, "ln_single.weight", dtype), _p(params, "ln_single.bias", dtype), eps
    )
    d = cs // n_head
    q = x @ _p(params, "to_query.weight", dtype).T + _p(params, "to_query.bias", dtype)
    k = x @ _p(params, "to_key.weight", dtype).T
    v = x @ _p(params, "to_value.weight", dtype).T

    def heads(t: Tensor) -> Tensor:
        return t.reshape(batch, n, n_head, d).permute(0, 2, 1, 3)

    zn = layer_norm(z, _p(params, "ln_pair.weight", dtype), None, eps)
    bias = torch.einsum("bijc,hc->bhij", zn, _p(params, "to_bias.weight", dtype))
    if extra_bias is not None:
        bias = bias + extra_bias.detach().to("cpu", dtype)
    keep = mask.to("cpu", torch.bool)[:, None, None, :]
    o = _masked_softmax_attention(heads(q), heads(k), heads(v), bias, keep, d**-0.5)
    o = o.permute(0, 2, 1, 3).reshape(batch, n, cs)
    empty = ~mask.to("cpu", torch.bool).any(dim=-1)
    o = torch.where(empty[:, None, None], torch.zeros_like(o), o)
    gate = torch.sigmoid(x @ _p(params, "to_gate.weight", dtype).T + gate_bias)
    return s + (gate * o) @ _p(params, "to_out.weight", dtype).T


def msa_pair_weighted_averaging(
    m: Tensor,
    z: Tensor,
    mask: Tensor,
    params: Params,
    *,
    n_head: int,
    eps: float = 1e-5,
    dtype: torch.dtype = torch.float32,
) -> Tensor:
    """MSA pair-weighted averaging (``legacy/attention.py:203-223``), residual included.

    ``m [B, S, N, c_m]``, ``z [B, N, N, c_z]``, key mask ``[B, N]``:
    ``x = LN_msa(m)``; ``w[h, i, :] = softmax_j(LN_pair(z)[i, j] . W_b[h])`` over valid keys j
    (one set of weights for every MSA row); ``o[s, i, h] = sum_j w[h, i, j] v[s, j, h]`` with
    ``v = x W_v^T``; ``m + (sigmoid(x W_g^T) * o) W_out^T``. A batch element without a valid key
    gets a zero update.
    """
    m = m.detach().to("cpu", dtype)
    z = z.detach().to("cpu", dtype)
    batch, depth, n, cm = m.shape
    x = layer_norm(m, _p(params, "ln_msa.weight", dtype), _p(params, "ln_msa.bias", dtype), eps)
    hd = params["to_value.weight"].shape[0]
    d = hd // n_head
    zn = layer_norm(z, _p(params, "ln_pair.weight", dtype), None, eps)
    logits = torch.einsum("bijc,hc->bhij", zn, _p(params, "to_bias.weight", dtype))
    keep = mask.to("cpu", torch.bool)[:, None, None, :]
    w = torch.softmax(logits.masked_fill(~keep, MASK_VALUE), dim=-1)
    v = (x @ _p(params, "to_value.weight", dtype).T).reshape(batch, depth, n, n_head, d)
    o = torch.einsum("bhij,bsjhc->bsihc", w, v).reshape(batch, depth, n, hd)
    empty = ~mask.to("cpu", torch.bool).any(dim=-1)
    o = torch.where(empty[:, None, None, None], torch.zeros_like(o), o)
    gate = torch.sigmoid(x @ _p(params, "to_gate.weight", dtype).T)
    return m + (gate * o) @ _p(params, "to_out.weight", dtype).T


def outer_product_mean(
    m: Tensor,
    rows_mask: Tensor,
    params: Params,
    *,
    count_offset: float | None = 1e-3,
    normalize_before_proj: bool = False,
    groups: int = 1,
    eps: float = 1e-5,
    product_norm_eps: float = 0.1,
    dtype: torch.dtype = torch.float32,
) -> Tensor:
    """Outer product mean, the raw update ``[B, N, N, c_z]`` (no residual).

    Follows the dense module of ``legacy/primitives.py:80-136`` one batch element at a time,
    with the engine's ``to_out.weight [c_z, G K K]`` turned back into the released
    ``output_w [(G,) K, K, c_z]`` (the inverse of ``legacy/released.py:248``):
    ``left / right = mask * (LN(m) W^T + b)`` (``primitives.py:83-86``); ungrouped, AF3's
    contraction and divisor of ``legacy/reference/attention.py:71-74`` (``count_offset`` =
    AF3's 1e-3, bias before the divide), the clamp ``max(n, 1)`` when ``count_offset`` is
    None, and the bias after the divide for ``normalize_before_proj`` (``primitives.py:
    123-132``); grouped (``primitives.py:138-156``): products within each group, summed over
    the MSA rows, ``product_norm``, projection, no divide.
    """
    m = m.detach().to("cpu", dtype)
    keep_all = rows_mask.detach().to("cpu", dtype)
    batch, depth, n, _ = m.shape
    x = layer_norm(m, _p(params, "ln_msa.weight", dtype), _p(params, "ln_msa.bias", dtype), eps)
    wl, wr = _p(params, "to_left.weight", dtype), _p(params, "to_right.weight", dtype)
    bl = _p(params, "to_left.bias", dtype) if "to_left.bias" in params else None
    br = _p(params, "to_right.bias", dtype) if "to_right.bias" in params else None
    wo, bo = _p(params, "to_out.weight", dtype), _p(params, "to_out.bias", dtype)
    cz = wo.shape[0]
    k = wl.shape[0] // groups
    out = []
    for b in range(batch):
        mask = keep_all[b][..., None]  # [S, N, 1]
        left = x[b] @ wl.T + (0 if bl is None else bl)
        right = x[b] @ wr.T + (0 if br is None else br)
        left, right = mask * left, mask * right
        if groups > 1:
            lg, rg = left.unflatten(-1, (groups, k)), right.unflatten(-1, (groups, k))
            product = torch.einsum("sigk,sjgl->ijgkl", lg, rg).flatten(-3)
            product = layer_norm(product, _p(params, "product_norm.weight", dtype),
                                 _p(params, "product_norm.bias", dtype), product_norm_eps)
            out.append(product @ wo.T.reshape(groups * k * k, cz) + bo)
            continue
        output_w = wo.T.reshape(k, k, cz)
        outer = torch.einsum("acb,ade->dceb", left.permute(0, 2, 1), right)
        output = torch.einsum("dceb,cef->dbf", outer, output_w)
        norm = torch.einsum("abc,adc->bdc", mask, mask)
        divisor = norm.clamp_min(1.0) if count_offset is None else norm + count_offset
        if normalize_before_proj:
            out.append(output.permute(1, 0, 2) / divisor + bo)
        else:
            out.append((output + bo).permute(1, 0, 2) / divisor)
    return torch.stack(out)


def sub_params(params: Params, prefix: str) -> dict[str, Tensor]:
    """The entries of ``params`` under ``prefix.`` with the prefix removed."""
    head = prefix + "."
    return {k[len(head) :]: v for k, v in params.items() if k.startswith(head)}


def pairformer_block(
    z: Tensor,
    mask: Tensor,
    params: Params,
    *,
    n_head_pair: int = 4,
    s: Tensor | None = None,
    n_head_single: int = 16,
    single_gate_bias: float = 0.0,
    extra_pair_bias: Tensor | None = None,
    transposed_bias: bool = False,
    eps: float = 1e-5,
    dtype: torch.dtype = torch.float32,
    io_dtype: torch.dtype | None = None,
    parallel: bool = False,
) -> Tensor | tuple[Tensor, Tensor]:
    """One Pairformer block: the sequential AF3 order (``legacy/pairformer.py:191-230``) or,
    with ``parallel``, the schedule of ``legacy/pairformer.py:176-190`` and ``:208-226``.

    Sequential: ``z <- TM_out(z); z <- TM_in(z); z <- TA_start(z); z <- TA_end(z); z <- Tr(z)``;
    with a single track ``s <- APB(s, z); s <- Tr_s(s)``.
    Parallel: every update reads the block's input ``z0`` (``s0``):
    ``z = z0 + (dTM_out + dTM_in + dTA_start + dTA_end) + dTr``, ``s = s0 + dAPB(s0, z0) +
    dTr_s(s0)``. ``params`` holds the block's engine keys (``tri_multi_outgoing.to_left.weight`` ...).
    ``extra_pair_bias`` (broadcast to ``[B, H, N, N]``) joins the single attention's logits
    (``legacy/pairformer.py:216-218``).

    ``io_dtype`` (e.g. bf16) rounds the residual stream to that dtype after every op, as
    an engine op returns ``x + f(x)`` in its input dtype (``README.md:143-145``; bf16
    activations, ``src/foldforge/modules/engine/configure.py:73-99``); the arithmetic
    inside each op stays in ``dtype``. None keeps the stream in ``dtype`` throughout.
    """
    kw = {"eps": eps, "dtype": dtype}

    def io(t: Tensor) -> Tensor:
        return t if io_dtype is None else t.to(io_dtype).to(dtype)

    if parallel:
        z0 = z.to(dtype)
        upd = (triangle_multiplication(z, mask, sub_params(params, "tri_multi_outgoing"), outgoing=True, **kw) - z0) \
            + (triangle_multiplication(z, mask, sub_params(params, "tri_multi_incoming"), outgoing=False, **kw) - z0)
        for name, starting in (("tri_atten_starting", True), ("tri_atten_ending", False)):
            if f"{name}.to_bias.weight" in params:
                upd = upd + (triangle_attention(z, mask, sub_params(params, name), starting=starting,
                                                n_head=n_head_pair, transposed_bias=transposed_bias, **kw) - z0)
        z_out = io(z0 + upd + (transition(z, sub_params(params, "transition_pair"), **kw) - z0))
        if s is None:
            return z_out
        s0 = s.to(dtype)
        ds = attention_pair_bias(s, z, mask, sub_params(params, "single_attention"), n_head=n_head_single,
                                 gate_bias=single_gate_bias, extra_bias=extra_pair_bias, **kw) - s0
        return z_out, io(s0 + ds + (transition(s, sub_params(params, "single_transition"), **kw) - s0))

    z = io(triangle_multiplication(
        z, mask, sub_params(params, "tri_multi_outgoing"), outgoing=True, **kw
    ))
    z = io(triangle_multiplication(
        z, mask, sub_params(params, "tri_multi_incoming"), outgoing=False, **kw
    ))
    z = io(triangle_attention(
        z, mask, sub_params(params, "tri_atten_starting"), starting=True,
        n_head=n_head_pair, transposed_bias=transposed_bias, **kw,
    ))
    z = io(triangle_attention(
        z, mask, sub_params(params, "tri_atten_ending"), starting=False,
        n_head=n_head_pair, transposed_bias=transposed_bias, **kw,
    ))
    z = io(transition(z, sub_params(params, "transition_pair"), **kw))
    if s is None:
        return z
    s = io(attention_pair_bias(
        s, z, mask, sub_params(params, "single_attention"), n_head=n_head_single,
        gate_bias=single_gate_bias, extra_bias=extra_pair_bias, **kw,
    ))
    s = io(transition(s, sub_params(params, "single_transition"), **kw))
    return z, s


def rel_rms(actual: Tensor, expected: Tensor, where: Tensor | None = None) -> float:
    """``||a - e||_2 / ||e||_2`` in fp64, over ``where`` when given."""
    a, e = actual.detach().double().cpu(), expected.detach().double().cpu()
    if where is not None:
        a, e = a[where], e[where]
    den = e.square().mean().sqrt().clamp_min(1e-30)
    return float((a - e).square().mean().sqrt() / den)


def max_abs(actual: Tensor, expected: Tensor, where: Tensor | None = None) -> float:
    a, e = actual.detach().double().cpu(), expected.detach().double().cpu()
    if where is not None:
        a, e = a[where], e[where]
    return float((a - e).abs().max()) if a.numel() else 0.0


def flops_triangle_attention_core(batch: int, n: int, heads: int, d: int) -> float:
    """``4 B N^3 H D``: Q K^T and P V over every row."""
    return 4.0 * batch * n**3 * heads * d


def flops_trimul_contraction(batch: int, n: int, hidden: int) -> float:
    return 2.0 * batch * n**3 * hidden

