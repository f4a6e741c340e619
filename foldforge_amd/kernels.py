"""Functional entry points of the HIP kernels, named after the engine's kernel functions.

The engine exposes ``layer_norm``, ``layer_norm_linear``, ``swiglu_ffn``,
``triangle_multiplicative_update``, ``triangle_attention`` and ``transition_layer`` under
``miniworld_engine.kernels`` (names: ``docs/guides/ENGINE-2.4.2.md:18-21`` of the reference;
their signatures are not in the reference, so these are this library's own); ``attention_pair_bias`` serves
the engine's ``single_attention`` op (``AttentionPairBias``) and
``msa_pair_weighted_averaging`` its ``msa_pwa`` op (``MSAPairWeightedAveraging``) and
``outer_product_mean`` its ``opm`` op (``OuterProductMean``). Each function validates its
tensors, allocates the output and the workspace with torch's allocator on the input's
device, and calls the C-ABI on torch's current stream. There is no fallback: the
module classes decide what to refuse (``unsupported``) before a call ever gets here.
"""

from __future__ import annotations

import torch

from foldforge_amd import _native

Tensor = torch.Tensor

PAIR_WIDTH = 128
TRI_HEADS = 4
TRI_HEAD_DIM = 32


#: The device type the kernels run on. Host-side argument checks compare against it, so a
#: CPU test can exercise them by pointing it at "cpu" (nothing reaches the library then:
#: every such test expects a ValueError before the native call).
DEVICE_TYPE = "cuda"


def _on_device(t: Tensor) -> bool:
    return t.device.type == DEVICE_TYPE


def _ptr(t: Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _need(cond: bool, message: str) -> None:
    if not cond:
        raise ValueError(message)


def _param(t: Tensor, device: torch.device, name: str, shape: tuple[int, ...] | None = None) -> Tensor:
    """An fp32 parameter on ``device`` of exactly ``shape``: the C-ABI receives no sizes for
    parameters, so a wrong shape must stop here, not as an out-of-bounds device read."""
    _need(isinstance(t, Tensor), f"{name} is missing")
    _need(t.device == device, f"{name} is on {t.device}, expected {device}")
    _need(t.dtype == torch.float32, f"{name} must be fp32 (got {t.dtype})")
    if shape is not None:
        _need(tuple(t.shape) == tuple(shape), f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    return t.contiguous()


def _output(out: Tensor | None, shape: tuple[int, ...], dtype: torch.dtype, device: torch.device) -> Tensor:
    """The caller's ``out=`` tensor (checked: it is written through a raw pointer) or a new one."""
    if out is None:
        return torch.empty(shape, dtype=dtype, device=device)
    _need(tuple(out.shape) == tuple(shape), f"out has shape {tuple(out.shape)}, expected {tuple(shape)}")
    _need(out.dtype == dtype, f"out must be {dtype} (got {out.dtype})")
    _need(out.device == device, f"out is on {out.device}, expected {device}")
    _need(out.is_contiguous(), "out must be contiguous")
    return out


def _workspace(nbytes: int, device: torch.device) -> Tensor:
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


def trimul_supported(d_pair: int, d_hidden: int) -> bool:
    """Widths of the triangle-multiplication kernels: the fused AF3 trunk kernels (128 / 128)
    or the generic path (pair a multiple of 64 up to 256, hidden a multiple of 64 up to 768)."""
    return (d_pair, d_hidden) == (128, 128) or (
        0 < d_pair <= 256 and d_pair % 64 == 0 and 0 < d_hidden <= 768 and d_hidden % 64 == 0)


def triangle_attention_supported(d_pair: int, n_head: int, d_head: int, transposed_bias: bool) -> bool:
    """Shapes of the triangle-attention kernels: the fused AF3 trunk kernels (128, 4 x 32) or
    the generic path (pair 64 / 128 / 256, at most 32 heads of 8 to 64 channels with
    heads x d_head a multiple of 64: the template stacks' and Chai-1's 4 x 64 on pair 256);
    both take either bias orientation and every output form."""
    if (d_pair, n_head, d_head) == (128, 4, 32):
        return True
    return (d_pair in (64, 128, 256) and 0 < n_head <= 32 and 0 < d_head <= 64 and d_head % 8 == 0
            and (n_head * d_head) % 64 == 0)


def _pair(z: Tensor, mask: Tensor, width: int | None = PAIR_WIDTH) -> tuple[int, int]:
    _need(_on_device(z), "z must be a device tensor")
    _need(z.dtype == torch.bfloat16, f"z must be bf16 (got {z.dtype})")
    _need(z.dim() == 4 and z.shape[1] == z.shape[2], f"z must be [B, N, N, c] (got {tuple(z.shape)})")
    if width is not None:
        _need(z.shape[3] == width, f"pair width {z.shape[3]} (the kernels take {width})")
    _need(z.is_contiguous(), "z must be contiguous")
    _need(mask.dtype == torch.bool and mask.shape == z.shape[:2], "mask must be bool [B, N]")
    _need(mask.device == z.device and mask.is_contiguous(), "mask must be a contiguous device tensor")
    return z.shape[0], z.shape[1]


def layer_norm(x: Tensor, weight: Tensor | None, bias: Tensor | None, eps: float = 1e-5) -> Tensor:
    """LayerNorm over the last axis (fp32 statistics and affine), returned in ``x.dtype``."""
    _need(_on_device(x) and x.is_contiguous(), "x must be a contiguous device tensor")
    _need(x.dtype in (torch.bfloat16, torch.float32), f"x must be bf16 or fp32 (got {x.dtype})")
    cols = x.shape[-1]
    for t, name in ((weight, "weight"), (bias, "bias")):
        if t is not None:
            _need(t.numel() == cols, f"{name} has {t.numel()} entries for {cols} channels")
    weight = None if weight is None else _param(weight, x.device, "weight", (cols,))
    bias = None if bias is None else _param(bias, x.device, "bias", (cols,))
    y = torch.empty_like(x)
    dtype = 0 if x.dtype == torch.bfloat16 else 1
    status = _native.lib().ffk_layer_norm(
        x.data_ptr(), _ptr(weight), _ptr(bias), y.data_ptr(), x.numel() // cols, cols,
        float(eps), dtype, _stream(x.device),
    )
    _native.check(status, "layer_norm")
    return y


#: ``layer_norm_linear`` activations -> the C-ABI's FFK_ACT_* values
ACTIVATIONS = {"none": 0, "sigmoid": 1, "silu": 2, "relu": 3}


def layer_norm_linear(x: Tensor, ln_weight: Tensor | None, ln_bias: Tensor | None, weight: Tensor,
                      bias: Tensor | None = None, *, activation: str = "none",
                      out_dtype: torch.dtype = torch.bfloat16, eps: float = 1e-5,
                      out: Tensor | None = None) -> Tensor:
    """``act(LN(x) W^T + b)`` over the last axis of ``x [..., d_in]`` bf16 (the engine's
    ``layer_norm_linear``): fp32 statistics, ``weight [d_out, d_in]`` fp32, ``bias [d_out]``,
    output ``[..., d_out]`` in ``out_dtype`` (bf16 or fp32). d_in a multiple of 64 up to 768,
    d_out a multiple of 32."""
    _need(_on_device(x) and x.is_contiguous(), "x must be a contiguous device tensor")
    _need(x.dtype == torch.bfloat16, f"x must be bf16 (got {x.dtype})")
    _need(activation in ACTIVATIONS, f"activation must be one of {sorted(ACTIVATIONS)}")
    _need(out_dtype in (torch.bfloat16, torch.float32), f"out_dtype must be bf16 or fp32 (got {out_dtype})")
    d_in = x.shape[-1]
    _need(weight.dim() == 2, f"weight must be [d_out, d_in] (got {tuple(weight.shape)})")
    d_out = weight.shape[0]
    _need(d_in % 64 == 0 and 0 < d_in <= 768 and d_out % 32 == 0 and d_out > 0,
          f"d_in={d_in} d_out={d_out} (the kernel takes d_in a multiple of 64 up to 768, d_out a multiple of 32)")
    dev = x.device
    w = _param(weight, dev, "weight", (d_out, d_in))
    lw = None if ln_weight is None else _param(ln_weight, dev, "ln_weight", (d_in,))
    lb = None if ln_bias is None else _param(ln_bias, dev, "ln_bias", (d_in,))
    b = None if bias is None else _param(bias, dev, "bias", (d_out,))
    out = _output(out, (*x.shape[:-1], d_out), out_dtype, dev)
    status = _native.lib().ffk_layer_norm_linear(
        x.data_ptr(), _ptr(lw), _ptr(lb), w.data_ptr(), _ptr(b), out.data_ptr(), x.numel() // d_in,
        d_in, d_out, ACTIVATIONS[activation], 0 if out_dtype == torch.bfloat16 else 1, float(eps),
        _stream(dev))
    _native.check(status, "layer_norm_linear")
    return out


def swiglu_ffn(x: Tensor, w_a: Tensor, w_b: Tensor, w_out: Tensor, residual: Tensor | None = None, *,
               out: Tensor | None = None) -> Tensor:
    """``(silu(x W_a^T) * (x W_b^T)) W_out^T`` (+ ``residual``) over the last axis of
    ``x [..., d]`` bf16 (the engine's ``swiglu_ffn``): ``w_a, w_b [hidden, d]``,
    ``w_out [d, hidden]`` fp32; d a multiple of 64 up to 768, hidden a multiple of 64."""
    _need(_on_device(x) and x.is_contiguous(), "x must be a contiguous device tensor")
    _need(x.dtype == torch.bfloat16, f"x must be bf16 (got {x.dtype})")
    d = x.shape[-1]
    hidden = w_a.shape[0]
    _need(d % 64 == 0 and 0 < d <= 768 and hidden % 64 == 0 and hidden > 0,
          f"d={d} hidden={hidden} (the kernel takes d a multiple of 64 up to 768, hidden a multiple of 64)")
    dev = x.device
    wa = _param(w_a, dev, "w_a", (hidden, d))
    wb = _param(w_b, dev, "w_b", (hidden, d))
    wo = _param(w_out, dev, "w_out", (d, hidden))
    if residual is not None:
        _need(residual.dtype == torch.bfloat16 and residual.shape == x.shape and residual.device == dev
              and residual.is_contiguous(), "residual must be a contiguous bf16 tensor shaped like x")
    out = _output(out, tuple(x.shape), torch.bfloat16, dev)
    rows = x.numel() // d
    lib = _native.lib()
    ws = _workspace(lib.ffk_swiglu_ffn_workspace(rows, hidden), dev)
    status = lib.ffk_swiglu_ffn(x.data_ptr(), wa.data_ptr(), wb.data_ptr(), wo.data_ptr(), _ptr(residual),
                                out.data_ptr(), ws.data_ptr(), ws.numel(), rows, d, hidden, _stream(dev))
    _native.check(status, "swiglu_ffn")
    return out


def triangle_multiplicative_update(
    z: Tensor,
    mask: Tensor,
    *,
    ln_pair_weight: Tensor,
    ln_pair_bias: Tensor,
    to_left: Tensor,
    to_right: Tensor,
    to_left_gate: Tensor,
    to_right_gate: Tensor,
    ln_out_weight: Tensor,
    ln_out_bias: Tensor,
    to_out: Tensor,
    to_gate: Tensor,
    outgoing: bool,
    residual: bool = True,
    length_divided: bool = False,
    eps: float = 1e-5,
    out: Tensor | None = None,
) -> Tensor:
    """Triangle multiplication (outgoing / incoming) of ``z [B, N, N, c]`` bf16 under the key mask.

    ``length_divided``: RoseTTAFold3's exact form, the contraction divided by the number of
    positions real in any batch element before the centre norm
    (``src/foldforge/models/checkpoints/legacy/routing.py:33-55``); the count stays on the device."""
    batch, n = _pair(z, mask, width=None)
    c = z.shape[3]
    dev = z.device
    hidden = to_left.shape[0]
    _need(trimul_supported(c, hidden), f"d_pair={c} d_hidden={hidden} (the kernels take 128 / 128, "
          "or a pair width a multiple of 64 up to 256 with a hidden width a multiple of 64 up to 768)")
    spec = (("ln_pair_weight", ln_pair_weight, (c,)), ("ln_pair_bias", ln_pair_bias, (c,)),
            ("to_left", to_left, (hidden, c)), ("to_right", to_right, (hidden, c)),
            ("to_left_gate", to_left_gate, (hidden, c)), ("to_right_gate", to_right_gate, (hidden, c)),
            ("ln_out_weight", ln_out_weight, (hidden,)), ("ln_out_bias", ln_out_bias, (hidden,)),
            ("to_out", to_out, (c, hidden)), ("to_gate", to_gate, (c, c)))
    ps = [_param(t, dev, nm, shape) for nm, t, shape in spec]
    out = _output(out, tuple(z.shape), torch.bfloat16, dev)
    lib = _native.lib()
    ws = _workspace(lib.ffk_triangle_multiplication_workspace(batch, n, c, hidden), dev)
    status = lib.ffk_triangle_multiplication(
        z.data_ptr(), mask.data_ptr(), *(p.data_ptr() for p in ps), out.data_ptr(),
        ws.data_ptr(), ws.numel(), batch, n, c, hidden, int(outgoing), int(residual),
        int(length_divided), float(eps), _stream(dev),
    )
    _native.check(status, "triangle_multiplicative_update")
    return out


def triangle_attention(
    z: Tensor,
    mask: Tensor,
    *,
    ln_pair_weight: Tensor,
    ln_pair_bias: Tensor,
    to_bias: Tensor,
    to_query: Tensor,
    to_key: Tensor,
    to_value: Tensor,
    to_gate: Tensor,
    to_out: Tensor,
    n_head: int,
    starting: bool,
    gate_bias: Tensor | None = None,
    out_bias: Tensor | None = None,
    to_out_t: Tensor | None = None,
    out_t_bias: Tensor | None = None,
    transposed_bias: bool = False,
    untransposed_output: bool = False,
    residual: bool = True,
    eps: float = 1e-5,
    out: Tensor | None = None,
) -> Tensor:
    """Triangle attention around the starting / ending node of ``z [B, N, N, c]`` bf16.

    ``gate_bias`` / ``out_bias``: RoseTTAFold3's projection biases. ``untransposed_output``:
    Chai-1's trunk, the ending node's update not turned back. ``to_out_t`` (+ ``out_t_bias``):
    Chai-1's confidence head, a second output projection added transposed over the pair axes."""
    batch, n = _pair(z, mask, width=None)
    c = z.shape[3]
    dev = z.device
    hd = to_query.shape[0]
    _need(n_head > 0 and hd % n_head == 0, f"hidden {hd} is not a multiple of {n_head} heads")
    _need(out_t_bias is None or to_out_t is not None, "out_t_bias needs to_out_t")
    spec = (("ln_pair_weight", ln_pair_weight, (c,)), ("ln_pair_bias", ln_pair_bias, (c,)),
            ("to_bias", to_bias, (n_head, c)), ("to_query", to_query, (hd, c)),
            ("to_key", to_key, (hd, c)), ("to_value", to_value, (hd, c)),
            ("to_gate", to_gate, (hd, c)), ("to_out", to_out, (c, hd)))
    ps = [_param(t, dev, nm, shape) for nm, t, shape in spec]
    extra = (("gate_bias", gate_bias, (hd,)), ("out_bias", out_bias, (c,)),
             ("to_out_t", to_out_t, (c, hd)), ("out_t_bias", out_t_bias, (c,)))
    opt = [None if t is None else _param(t, dev, nm, shape) for nm, t, shape in extra]
    # the starting node's untransposed update is the standard one: asking for form 0 spares the
    # workspace the staging buffer of form 1
    form = 2 if to_out_t is not None else 1 if untransposed_output and not starting else 0
    d = hd // n_head
    _need(triangle_attention_supported(c, n_head, d, transposed_bias),
          f"d_pair={c} heads={n_head} x {d} (the kernels take 128 with 4 x 32, or pair 64 / 128 / "
          "256 with at most 32 heads of 8 to 64 channels, heads x d_head a multiple of 64)")
    if (c, n_head, d) != (128, 4, 32):
        _need(batch * n <= 65535, f"batch x n = {batch * n} exceeds the launch grid")
    out = _output(out, tuple(z.shape), torch.bfloat16, dev)
    lib = _native.lib()
    ws = _workspace(lib.ffk_triangle_attention_workspace(batch, n, c, n_head, d, form), dev)
    status = lib.ffk_triangle_attention(
        z.data_ptr(), mask.data_ptr(), *(p.data_ptr() for p in ps), *(_ptr(t) for t in opt),
        out.data_ptr(), ws.data_ptr(), ws.numel(), batch, n, c, n_head, d, int(starting),
        int(transposed_bias), form, int(residual), float(eps), _stream(dev),
    )
    _native.check(status, "triangle_attention")
    return out


def transition(
    x: Tensor,
    *,
    ln_weight: Tensor,
    ln_bias: Tensor,
    expand_a: Tensor,
    expand_b: Tensor,
    squeeze: Tensor,
    residual: bool = True,
    eps: float = 1e-5,
    out: Tensor | None = None,
) -> Tensor:
    """SwiGLU transition of ``x [..., d]`` bf16: one fused kernel at d = 128 x 4, token-row
    GEMMs (LayerNorm, expand with SwiGLU epilogue, squeeze + residual) at other widths."""
    _need(_on_device(x) and x.is_contiguous(), "x must be a contiguous device tensor")
    _need(x.dtype == torch.bfloat16, f"x must be bf16 (got {x.dtype})")
    d = x.shape[-1]
    factor = expand_a.shape[0] // d
    _need(transition_supported(d, factor),
          f"width {d} x {factor} (the kernels take 128 x 4, or d and factor * d multiples of 64)")
    _need(expand_a.shape == (factor * d, d) and expand_b.shape == (factor * d, d)
          and squeeze.shape == (d, factor * d), "expand_a/expand_b [f d, d], squeeze [d, f d]")
    dev = x.device
    spec = (("ln_weight", ln_weight, (d,)), ("ln_bias", ln_bias, (d,)),
            ("expand_a", expand_a, (factor * d, d)), ("expand_b", expand_b, (factor * d, d)),
            ("squeeze", squeeze, (d, factor * d)))
    ps = [_param(t, dev, nm, shape) for nm, t, shape in spec]
    rows = x.numel() // d
    out = _output(out, tuple(x.shape), torch.bfloat16, dev)
    lib = _native.lib()
    ws = _workspace(lib.ffk_transition_workspace(rows, d, factor), dev)
    status = lib.ffk_transition(
        x.data_ptr(), *(p.data_ptr() for p in ps), out.data_ptr(), ws.data_ptr(), ws.numel(),
        rows, d, factor, int(residual), float(eps), _stream(dev),
    )
    _native.check(status, "transition")
    return out


#: the engine's name for the transition kernel (``docs/guides/ENGINE-2.4.2.md:19``)
transition_layer = transition


def triangle_attention_transition(
    z: Tensor,
    mask: Tensor,
    *,
    ln_pair_weight: Tensor,
    ln_pair_bias: Tensor,
    to_bias: Tensor,
    to_query: Tensor,
    to_key: Tensor,
    to_value: Tensor,
    to_gate: Tensor,
    to_out: Tensor,
    ln_weight: Tensor,
    ln_bias: Tensor,
    expand_a: Tensor,
    expand_b: Tensor,
    squeeze: Tensor,
    starting: bool = False,
    transposed_bias: bool = False,
    eps_pair: float = 1e-5,
    eps: float = 1e-5,
    out: Tensor | None = None,
) -> Tensor:
    """``transition(triangle_attention(z))`` with both residuals, the attention's gate and
    output projection computed inside the transition kernel (the attention's output never
    reaches HBM): the last two pair updates of a sequential Pairformer block
    (``legacy/pairformer.py:200-202``). AF3 trunk widths only (pair 128, 4 heads x 32,
    transition 128 x 4), no gate / output projection biases."""
    batch, n = _pair(z, mask)
    dev = z.device
    c, hd = PAIR_WIDTH, TRI_HEADS * TRI_HEAD_DIM
    spec = (("ln_pair_weight", ln_pair_weight, (c,)), ("ln_pair_bias", ln_pair_bias, (c,)),
            ("to_bias", to_bias, (TRI_HEADS, c)), ("to_query", to_query, (hd, c)),
            ("to_key", to_key, (hd, c)), ("to_value", to_value, (hd, c)),
            ("to_gate", to_gate, (hd, c)), ("to_out", to_out, (c, hd)),
            ("ln_weight", ln_weight, (c,)), ("ln_bias", ln_bias, (c,)),
            ("expand_a", expand_a, (4 * c, c)), ("expand_b", expand_b, (4 * c, c)),
            ("squeeze", squeeze, (c, 4 * c)))
    ps = [_param(t, dev, nm, shape) for nm, t, shape in spec]
    out = _output(out, tuple(z.shape), torch.bfloat16, dev)
    lib = _native.lib()
    ws = _workspace(lib.ffk_triangle_attention_transition_workspace(batch, n), dev)
    status = lib.ffk_triangle_attention_transition(
        z.data_ptr(), mask.data_ptr(), *(p.data_ptr() for p in ps), out.data_ptr(),
        ws.data_ptr(), ws.numel(), batch, n, int(starting), int(transposed_bias),
        float(eps_pair), float(eps), _stream(dev),
    )
    _native.check(status, "triangle_attention_transition")
    return out


def transition_supported(d: int, factor: int) -> bool:
    """Widths the transition kernels take."""
    return (d == PAIR_WIDTH and factor == 4) or (d > 0 and factor > 0 and d % 64 == 0
                                                 and (factor * d) % 64 == 0)


def single_attention_heads_supported(d_single: int, n_head: int) -> bool:
    """Single widths and head splits the attention-with-pair-bias kernels take."""
    if n_head <= 0 or n_head > 32 or d_single <= 0 or d_single % 64 or d_single % n_head:
        return False
    dh = d_single // n_head
    return dh % 8 == 0 and dh <= 32


def attention_pair_bias(
    s: Tensor,
    z: Tensor,
    mask: Tensor,
    *,
    ln_single_weight: Tensor,
    ln_single_bias: Tensor,
    to_query: Tensor,
    query_bias: Tensor,
    to_key: Tensor,
    to_value: Tensor,
    ln_pair_weight: Tensor,
    to_bias: Tensor,
    to_gate: Tensor,
    to_out: Tensor,
    n_head: int,
    gate_bias: float = 0.0,
    extra_bias: Tensor | None = None,
    residual: bool = True,
    eps_single: float = 1e-5,
    eps_pair: float = 1e-5,
    out: Tensor | None = None,
) -> Tensor:
    """Single-track attention with pair bias: ``s [B, N, c_s]`` bf16 attends over tokens with
    the bias ``LN_pair(z) . to_bias`` from ``z [B, N, N, 128]`` bf16, under the key mask.
    ``extra_bias`` (fp32 or bf16, broadcastable to ``[B, H, N, N]``, e.g. an ``[N, N]`` or
    an expanded view) joins every logit; broadcast axes are passed as zero strides."""
    batch, n = _pair(z, mask)
    _need(_on_device(s) and s.is_contiguous() and s.dtype == torch.bfloat16,
          "s must be a contiguous bf16 device tensor")
    _need(s.dim() == 3 and s.shape[:2] == z.shape[:2], f"s {tuple(s.shape)} does not match z")
    cs = s.shape[-1]
    _need(single_attention_heads_supported(cs, n_head),
          f"single width {cs} with {n_head} heads (the kernels take a multiple of 64 split "
          "into at most 32 heads of 8, 16, 24 or 32)")
    dev = s.device
    spec = (("ln_single_weight", ln_single_weight, (cs,)), ("ln_single_bias", ln_single_bias, (cs,)),
            ("to_query", to_query, (cs, cs)), ("query_bias", query_bias, (cs,)),
            ("to_key", to_key, (cs, cs)), ("to_value", to_value, (cs, cs)),
            ("ln_pair_weight", ln_pair_weight, (PAIR_WIDTH,)), ("to_bias", to_bias, (n_head, PAIR_WIDTH)),
            ("to_gate", to_gate, (cs, cs)), ("to_out", to_out, (cs, cs)))
    ps = [_param(t, dev, nm, shape) for nm, t, shape in spec]
    extra, strides, extra_bf16 = None, (0, 0, 0), 0
    if extra_bias is not None:
        _need(extra_bias.dtype in (torch.float32, torch.bfloat16),
              f"extra_bias must be fp32 or bf16 (got {extra_bias.dtype})")
        _need(extra_bias.device == dev, "extra_bias must be on the device of s")
        try:
            extra = extra_bias.expand(batch, n_head, n, n)
        except RuntimeError:
            raise ValueError(f"extra_bias {tuple(extra_bias.shape)} does not broadcast to "
                             f"{(batch, n_head, n, n)}") from None
        if extra.stride(-1) != 1:
            extra = extra.contiguous()
        strides, extra_bf16 = extra.stride()[:3], int(extra.dtype == torch.bfloat16)
    out = _output(out, tuple(s.shape), torch.bfloat16, dev)
    lib = _native.lib()
    ws = _workspace(lib.ffk_attention_pair_bias_workspace(batch, n, cs, PAIR_WIDTH, n_head), dev)
    status = lib.ffk_attention_pair_bias(
        s.data_ptr(), z.data_ptr(), mask.data_ptr(), *(p.data_ptr() for p in ps), _ptr(extra),
        extra_bf16, *strides, out.data_ptr(), ws.data_ptr(), ws.numel(), batch, n, cs,
        PAIR_WIDTH, n_head, float(gate_bias), int(residual), float(eps_single), float(eps_pair),
        _stream(dev),
    )
    _native.check(status, "attention_pair_bias")
    return out


def msa_pair_weighted_averaging_supported(d_msa: int, n_head: int, d_head: int) -> bool:
    """MSA widths and head splits the pair-weighted averaging kernels take."""
    return (0 < d_msa <= 768 and d_msa % 64 == 0 and 0 < n_head <= 32 and d_head > 0
            and d_head % 4 == 0 and (n_head * d_head) % 64 == 0 and n_head * d_head <= 768)


def msa_pair_weighted_averaging(
    m: Tensor,
    z: Tensor,
    mask: Tensor,
    *,
    ln_msa_weight: Tensor,
    ln_msa_bias: Tensor,
    ln_pair_weight: Tensor,
    to_bias: Tensor,
    to_value: Tensor,
    to_gate: Tensor,
    to_out: Tensor,
    n_head: int,
    residual: bool = True,
    eps_msa: float = 1e-5,
    eps_pair: float = 1e-5,
    out: Tensor | None = None,
) -> Tensor:
    """MSA pair-weighted averaging of ``m [B, S, N, c_m]`` bf16 with the weights
    ``softmax_j(LN_pair(z) . to_bias)`` from ``z [B, N, N, 128]`` bf16, under the key mask."""
    batch, n = _pair(z, mask)
    _need(_on_device(m) and m.is_contiguous() and m.dtype == torch.bfloat16,
          "m must be a contiguous bf16 device tensor")
    _need(m.dim() == 4 and m.shape[0] == batch and m.shape[2] == n,
          f"m {tuple(m.shape)} does not match z {tuple(z.shape)}")
    depth, cm = m.shape[1], m.shape[3]
    hd = to_value.shape[0]
    _need(hd % n_head == 0, f"hidden {hd} is not a multiple of {n_head} heads")
    dh = hd // n_head
    _need(msa_pair_weighted_averaging_supported(cm, n_head, dh),
          f"d_msa={cm} heads={n_head} x {dh} (the kernels take d_msa a multiple of 64 up to 768, "
          "at most 32 heads of a multiple of 4, heads x d_head a multiple of 64)")
    dev = m.device
    spec = (("ln_msa_weight", ln_msa_weight, (cm,)), ("ln_msa_bias", ln_msa_bias, (cm,)),
            ("ln_pair_weight", ln_pair_weight, (PAIR_WIDTH,)), ("to_bias", to_bias, (n_head, PAIR_WIDTH)),
            ("to_value", to_value, (hd, cm)), ("to_gate", to_gate, (hd, cm)), ("to_out", to_out, (cm, hd)))
    ps = [_param(t, dev, nm, shape) for nm, t, shape in spec]
    out = _output(out, tuple(m.shape), torch.bfloat16, dev)
    lib = _native.lib()
    ws = _workspace(lib.ffk_msa_pair_weighted_averaging_workspace(batch, depth, n, cm, PAIR_WIDTH,
                                                                  n_head, dh), dev)
    status = lib.ffk_msa_pair_weighted_averaging(
        m.data_ptr(), z.data_ptr(), mask.data_ptr(), *(p.data_ptr() for p in ps), out.data_ptr(),
        ws.data_ptr(), ws.numel(), batch, depth, n, cm, PAIR_WIDTH, n_head, dh, int(residual),
        float(eps_msa), float(eps_pair), _stream(dev),
    )
    _native.check(status, "msa_pair_weighted_averaging")
    return out


def outer_product_mean_supported(d_msa: int, d_hidden: int, d_pair: int) -> bool:
    """Widths the outer-product-mean kernels take."""
    return 0 < d_msa <= 768 and d_msa % 64 == 0 and d_hidden == 32 and d_pair == PAIR_WIDTH


def outer_product_mean(
    m: Tensor,
    rows_mask: Tensor,
    *,
    ln_weight: Tensor,
    ln_bias: Tensor,
    to_left: Tensor,
    to_right: Tensor,
    to_out: Tensor,
    to_out_bias: Tensor,
    left_bias: Tensor | None = None,
    right_bias: Tensor | None = None,
    residual: Tensor | None = None,
    count_offset: float | None = 1e-3,
    normalize_before_proj: bool = False,
    eps: float = 1e-5,
    out: Tensor | None = None,
) -> Tensor:
    """Outer product mean of ``m [B, S, N, c_m]`` bf16 under the MSA row mask
    ``rows_mask [B, S, N]`` bool -> ``[B, N, N, 128]`` bf16 (plus ``residual`` when given).
    ``count_offset`` None divides by ``max(n, 1)``, a number by ``n + count_offset``."""
    _need(_on_device(m) and m.is_contiguous() and m.dtype == torch.bfloat16,
          "m must be a contiguous bf16 device tensor")
    _need(m.dim() == 4, f"m must be [B, S, N, c_m] (got {tuple(m.shape)})")
    batch, depth, n, cm = m.shape
    _need(rows_mask.dtype == torch.bool and tuple(rows_mask.shape) == (batch, depth, n)
          and rows_mask.device == m.device and rows_mask.is_contiguous(),
          "rows_mask must be a contiguous bool device tensor [B, S, N]")
    hidden = to_left.shape[0]
    cz = to_out.shape[0]
    _need(outer_product_mean_supported(cm, hidden, cz),
          f"d_msa={cm} d_hidden={hidden} d_pair={cz} (the kernels take d_msa a multiple of 64 "
          "up to 768, d_hidden 32, d_pair 128)")
    _need(depth > 0 and n > 0 and batch > 0, "empty MSA")
    dev = m.device
    spec = (("ln_weight", ln_weight, (cm,)), ("ln_bias", ln_bias, (cm,)),
            ("to_left", to_left, (hidden, cm)), ("to_right", to_right, (hidden, cm)),
            ("to_out", to_out, (cz, hidden * hidden)), ("to_out_bias", to_out_bias, (cz,)))
    ln_w, ln_b, wl, wr, wo, bo = (_param(t, dev, nm, shape) for nm, t, shape in spec)
    bl = None if left_bias is None else _param(left_bias, dev, "left_bias", (hidden,))
    br = None if right_bias is None else _param(right_bias, dev, "right_bias", (hidden,))
    if residual is not None:
        _need(residual.dtype == torch.bfloat16 and residual.is_contiguous()
              and tuple(residual.shape) == (batch, n, n, cz) and residual.device == dev,
              "residual must be a contiguous bf16 [B, N, N, 128] device tensor")
    out = _output(out, (batch, n, n, cz), torch.bfloat16, dev)
    lib = _native.lib()
    ws = _workspace(lib.ffk_outer_product_mean_workspace(batch, depth, n, cm, hidden, cz), dev)
    status = lib.ffk_outer_product_mean(
        m.data_ptr(), rows_mask.data_ptr(), ln_w.data_ptr(), ln_b.data_ptr(), wl.data_ptr(),
        None if bl is None else bl.data_ptr(), wr.data_ptr(), None if br is None else br.data_ptr(),
        wo.data_ptr(), bo.data_ptr(), None if residual is None else residual.data_ptr(),
        out.data_ptr(), ws.data_ptr(), ws.numel(), batch, depth, n, cm, hidden, cz, float(eps),
        -1.0 if count_offset is None else float(count_offset), int(normalize_before_proj),
        _stream(dev),
    )
    _native.check(status, "outer_product_mean")
    return out


def outer_product_mean_grouped_supported(d_msa: int, groups: int, d_group: int, d_pair: int) -> bool:
    """Widths the grouped (Chai-1) outer-product-mean kernels take."""
    return 0 < d_msa <= 768 and d_msa % 64 == 0 and groups == 8 and d_group == 8 and d_pair in (128, 256)


def outer_product_mean_grouped(
    m: Tensor,
    rows_mask: Tensor,
    *,
    groups: int,
    ln_weight: Tensor,
    ln_bias: Tensor,
    to_left: Tensor,
    to_right: Tensor,
    norm_weight: Tensor,
    norm_bias: Tensor,
    to_out: Tensor,
    to_out_bias: Tensor,
    left_bias: Tensor | None = None,
    right_bias: Tensor | None = None,
    residual: Tensor | None = None,
    eps: float = 1e-5,
    norm_eps: float = 0.1,
    out: Tensor | None = None,
) -> Tensor:
    """Chai-1's grouped outer product mean of ``m [B, S, N, c_m]`` bf16 under ``rows_mask
    [B, S, N]`` bool -> ``[B, N, N, c_z]`` bf16: products within each of ``groups`` channel
    groups, summed over the MSA rows, the product norm (``norm_weight`` / ``norm_bias``, eps
    ``norm_eps``), then ``to_out`` (plus ``residual`` when given)."""
    _need(_on_device(m) and m.is_contiguous() and m.dtype == torch.bfloat16,
          "m must be a contiguous bf16 device tensor")
    _need(m.dim() == 4, f"m must be [B, S, N, c_m] (got {tuple(m.shape)})")
    batch, depth, n, cm = m.shape
    _need(rows_mask.dtype == torch.bool and tuple(rows_mask.shape) == (batch, depth, n)
          and rows_mask.device == m.device and rows_mask.is_contiguous(),
          "rows_mask must be a contiguous bool device tensor [B, S, N]")
    hidden = to_left.shape[0]
    cz = to_out.shape[0]
    _need(hidden % groups == 0, f"d_hidden={hidden} is not a multiple of groups={groups}")
    dg = hidden // groups
    _need(outer_product_mean_grouped_supported(cm, groups, dg, cz),
          f"d_msa={cm} {groups} groups of {dg} d_pair={cz} (the kernels take d_msa a multiple of "
          "64 up to 768, 8 groups of 8, d_pair 128 or 256)")
    _need(depth > 0 and n > 0 and batch > 0, "empty MSA")
    dev = m.device
    k2 = groups * dg * dg
    spec = (("ln_weight", ln_weight, (cm,)), ("ln_bias", ln_bias, (cm,)),
            ("to_left", to_left, (hidden, cm)), ("to_right", to_right, (hidden, cm)),
            ("norm_weight", norm_weight, (k2,)), ("norm_bias", norm_bias, (k2,)),
            ("to_out", to_out, (cz, k2)), ("to_out_bias", to_out_bias, (cz,)))
    ln_w, ln_b, wl, wr, nw, nb, wo, bo = (_param(t, dev, nm, shape) for nm, t, shape in spec)
    bl = None if left_bias is None else _param(left_bias, dev, "left_bias", (hidden,))
    br = None if right_bias is None else _param(right_bias, dev, "right_bias", (hidden,))
    if residual is not None:
        _need(residual.dtype == torch.bfloat16 and residual.is_contiguous()
              and tuple(residual.shape) == (batch, n, n, cz) and residual.device == dev,
              f"residual must be a contiguous bf16 [B, N, N, {cz}] device tensor")
    out = _output(out, (batch, n, n, cz), torch.bfloat16, dev)
    lib = _native.lib()
    ws = _workspace(lib.ffk_outer_product_mean_grouped_workspace(batch, depth, n, cm, groups, dg, cz), dev)
    status = lib.ffk_outer_product_mean_grouped(
        m.data_ptr(), rows_mask.data_ptr(), ln_w.data_ptr(), ln_b.data_ptr(), wl.data_ptr(),
        None if bl is None else bl.data_ptr(), wr.data_ptr(), None if br is None else br.data_ptr(),
        nw.data_ptr(), nb.data_ptr(), wo.data_ptr(), bo.data_ptr(),
        None if residual is None else residual.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(),
        batch, depth, n, cm, groups, dg, cz, float(eps), float(norm_eps), _stream(dev),
    )
    _native.check(status, "outer_product_mean_grouped")
    return out


def blocked_bias(bias: Tensor) -> Tensor:
    """``bias [B, H, Np, Np]`` (query, key; log2 units) -> the flash kernel's blocked fp32 layout
    ``[B * H, Np/32, Np/32, 4, 64, 4]``: entry ``[.., qb, kb, v, lane, e]`` with
    ``lane = 32 g + li`` is query ``32 qb + li``, key ``32 kb + 8 v + 4 g + e``."""
    b, h, n1, n2 = bias.shape
    _need(n1 == n2 and n1 % 32 == 0, "bias must be [B, H, Np, Np] with Np % 32 == 0")
    nb = n1 // 32
    t = bias.float().reshape(b * h, nb, 32, nb, 4, 2, 4)  # [bh, qb, li, kb, v, g, e]
    return t.permute(0, 1, 3, 4, 5, 2, 6).reshape(b * h, nb, nb, 4, 64, 4).contiguous()


def flash_v_layout(v_t: Tensor) -> Tensor:
    """``v_t [..., 32, Np]`` -> the flash kernel's v^T layout ``[..., Np / 32, 32, 32]``: blocked
    by 32 keys (block ``kb`` holds ``[d][keys 32 kb ..]``), and inside every group of 16 keys
    the keys stored in the order 0-3, 8-11, 4-7, 12-15 (index bits 2 and 3 exchanged)."""
    n = v_t.shape[-1]
    _need(n % 32 == 0, "the key count must be a multiple of 32")
    idx = torch.arange(n, device=v_t.device)
    perm = (idx & ~12) | ((idx & 4) << 1) | ((idx & 8) >> 1)
    d = v_t.shape[-2]
    blocked = v_t[..., perm].unflatten(-1, (n // 32, 32)).transpose(-3, -2)  # [..., Np/32, d, 32]
    _need(blocked.shape[-2] == d, "v_t must be [..., d, Np]")
    return blocked.contiguous()


def flash_attention_bias(
    q: Tensor,
    k: Tensor,
    v_t: Tensor,
    bias_blk: Tensor,
    out: Tensor,
    *,
    rows_valid: int,
    n_valid: int,
) -> Tensor:
    """The flash core on prepared operands (see ``ffk_flash_attention_bias``).

    ``q, k [B, H, R, Np, 32]`` bf16 (q pre-scaled by ``d^-1/2 log2 e``),
    ``v_t [B, H, R, Np / 32, 32, 32]`` bf16 from :func:`flash_v_layout`, ``bias_blk`` from
    :func:`blocked_bias`;
    ``out [B, R, n_valid, H * 32]`` bf16 receives ``o`` for rows < rows_valid.
    """
    batch, heads, rows, n_pad, d = q.shape
    _need(d == TRI_HEAD_DIM, f"head dim {d} (the kernel takes {TRI_HEAD_DIM})")
    _need(k.shape == q.shape and v_t.shape == (batch, heads, rows, n_pad // 32, d, 32), "q/k/v_t shapes")
    _need(bias_blk.dtype == torch.float32 and bias_blk.numel() == batch * heads * n_pad * n_pad,
          "bias_blk must be the blocked fp32 layout of [B, H, Np, Np]")
    _need(all(t.is_contiguous() for t in (q, k, v_t, bias_blk)), "operands must be contiguous")
    _need(out.dtype == torch.bfloat16 and out.dim() == 4 and out.shape[-1] == heads * d,
          "out must be bf16 [B, R, n_valid, H * 32]")
    _need(out.device == q.device and out.stride(3) == 1, "out must be on q's device with unit channel stride")
    _need(0 <= rows_valid <= rows and 0 <= n_valid <= n_pad, "valid extents exceed the operands")
    _need(out.shape[0] >= batch and out.shape[1] >= rows_valid and out.shape[2] >= n_valid,
          f"out {tuple(out.shape)} does not cover [{batch}, {rows_valid}, {n_valid}, {heads * d}]")
    _need(all(t.device == q.device for t in (k, v_t, bias_blk)), "operands must share q's device")
    status = _native.lib().ffk_flash_attention_bias(
        q.data_ptr(), k.data_ptr(), v_t.data_ptr(), bias_blk.data_ptr(), out.data_ptr(),
        batch, heads, rows, n_pad, rows_valid, n_valid,
        out.stride(0), out.stride(1), out.stride(2), _stream(q.device),
    )
    _native.check(status, "flash_attention_bias")
    return out
