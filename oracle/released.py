"""fp64 CPU restatement of the RELEASED-layout modules (test oracle for the weight conversion).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``). The AlphaFold 3 family's released
parameters carry the dense graph's names and layouts; ``foldforge_amd.released`` turns them
into the engine modules' state dicts. These functions compute each op straight from the
released names and layouts (unbatched, as the dense modules run), so that a converted engine
module can be checked against the released computation (the reference's own check:
``tests/kernels/test_released_conversions.py:55-160``).

Followed (paths relative to the reference tree, under ``src/foldforge/models/checkpoints/``):

* triangle multiplication: ``legacy/reference/triangle.py:19-49`` -- one projection and one
  gate of ``2 h`` rows with the two branches interleaved per hidden channel (row ``2 k`` =
  branch a, ``2 k + 1`` = branch b), the pair mask applied before the gate, outgoing
  ``"cik,cjk->cij"``, incoming ``"ckj,cki->cij"``;
* grid self-attention (triangle attention): ``legacy/attention.py:60-171`` (AF3 spec: bias
  from the un-transposed pair, output turned back), attention per
  ``legacy/reference/attention.py:77-100`` with the pair mask's row as key mask;
* transition: ``legacy/primitives.py:20-37`` with ``legacy/routing.py:62-76`` -- one
  ``transition1`` of ``2 n c`` rows split by ``chunk(2)`` into the SwiGLU halves;
* MSA attention (pair-weighted averaging): ``legacy/attention.py:174-229`` -- the pair norm
  WITH its offset, keys masked by ``1e9 * (max_s msa_mask - 1)``;
* outer product mean: ``legacy/primitives.py:80-136`` and ``legacy/reference/attention.py:
  57-74`` -- ``output_w [K, K, c_z]``, AF3 divisor ``n + 1e-3``;
* the pairformer's single attention: ``legacy/pairformer.py:204-229`` and
  ``legacy/transformer.py:93-137`` -- the pair-logit norm WITH its offset.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

Tensor = torch.Tensor
State = dict[str, Tensor]
F64 = torch.float64


def _sub(state: State, prefix: str) -> State:
    head = prefix + "."
    return {k[len(head):]: v.to(F64) for k, v in state.items() if k.startswith(head)}


def _f64(s: State) -> State:
    return {k: v.to(F64) for k, v in s.items()}


def _ln(x: Tensor, s: State, key: str, eps: float = 1e-5) -> Tensor:
    return F.layer_norm(x, x.shape[-1:], s[f"{key}.weight"], s.get(f"{key}.bias"), eps)


def _lin(x: Tensor, s: State, key: str) -> Tensor:
    return F.linear(x, s[f"{key}.weight"], s.get(f"{key}.bias"))


def triangle_multiplication(z: Tensor, pair_mask: Tensor, s: State, *, outgoing: bool) -> Tensor:
    """``z [N, N, c]``, ``pair_mask [N, N]`` -> ``z + update``."""
    s = _f64(s)
    z = z.to(F64)
    value = _ln(z, s, "left_norm_input")
    projection = _lin(value, s, "projection").movedim(-1, -3) * pair_mask.to(F64)[None]
    projection = projection * torch.sigmoid(_lin(value, s, "gate").movedim(-1, -3))
    a, b = projection.unflatten(-3, (-1, 2)).unbind(-3)
    equation = "cik,cjk->cij" if outgoing else "ckj,cki->cij"
    contracted = torch.einsum(equation, a, b).movedim(-3, -1)
    update = _lin(_ln(contracted, s, "center_norm"), s, "output_projection")
    return z + update * torch.sigmoid(_lin(value, s, "gating_linear"))


def triangle_attention(z: Tensor, pair_mask: Tensor, s: State, *, n_head: int, ending: bool) -> Tensor:
    """AF3 grid self-attention: ``z [N, N, c]``, ``pair_mask [N, N]`` -> ``z + update``."""
    s = _f64(s)
    z = z.to(F64)
    pair = _ln(z, s, "act_norm")
    bias = _lin(pair, s, "pair_bias_projection").permute(2, 0, 1)  # [H, N, N], un-transposed
    if ending:
        pair = pair.permute(1, 0, 2)
        pair_mask = pair_mask.transpose(0, 1)
    rows, n, _ = pair.shape

    def heads(t: Tensor) -> Tensor:
        return t.reshape(rows, n, n_head, -1).permute(0, 2, 1, 3)  # [rows, H, n, d]

    q, k, v = (heads(_lin(pair, s, f"{x}_projection")) for x in ("q", "k", "v"))
    logits = (q * q.shape[-1] ** -0.5) @ k.transpose(-1, -2) + bias[None]
    logits = logits.masked_fill(~pair_mask.bool()[:, None, None, :], -1e9)
    o = (torch.softmax(logits, dim=-1) @ v).permute(0, 2, 1, 3).reshape(rows, n, -1)
    out = _lin(torch.sigmoid(_lin(pair, s, "gating_query")) * o, s, "output_projection")
    if ending:
        out = out.permute(1, 0, 2)
    return z + out


def transition(x: Tensor, s: State) -> Tensor:
    s = _f64(s)
    x = x.to(F64)
    a, b = _lin(_ln(x, s, "input_layer_norm"), s, "transition1").chunk(2, dim=-1)
    return x + _lin(F.silu(a) * b, s, "transition2")


def msa_attention(msa: Tensor, msa_mask: Tensor, pair: Tensor, s: State, *, n_head: int) -> Tensor:
    """``msa [S, N, c_m]``, ``msa_mask [S, N]``, ``pair [N, N, c_z]`` -> ``msa + update``."""
    s = _f64(s)
    msa, pair = msa.to(F64), pair.to(F64)
    x = _ln(msa, s, "act_norm")
    logits = _lin(_ln(pair, s, "pair_norm"), s, "pair_logits").permute(2, 0, 1)
    logits = logits + 1e9 * (msa_mask.to(F64).max(dim=0).values - 1.0)
    weights = torch.softmax(logits, dim=-1)
    v = _lin(x, s, "v_projection").unflatten(-1, (n_head, -1))
    avg = torch.einsum("hqk,bkhc->bqhc", weights, v).flatten(-2)
    return msa + _lin(torch.sigmoid(_lin(x, s, "gating_query")) * avg, s, "output_projection")


def outer_product_mean(msa: Tensor, mask: Tensor, s: State, *, eps: float = 1e-3) -> Tensor:
    """AF3's outer product mean from ``output_w [K, K, c_z]`` -> the update ``[N, N, c_z]``."""
    s = _f64(s)
    x = _ln(msa.to(F64), s, "layer_norm_input")
    m = mask.to(F64)[..., None]
    left, right = m * _lin(x, s, "left_projection"), m * _lin(x, s, "right_projection")
    outer = torch.einsum("acb,ade->dceb", left.permute(0, 2, 1), right)
    output = torch.einsum("dceb,cef->dbf", outer, s["output_w"]) + s["output_b"]
    norm = torch.einsum("abc,adc->bdc", m, m)
    return output.permute(1, 0, 2) / (eps + norm)


def single_attention(single: Tensor, pair: Tensor, token_mask: Tensor, s: State, *,
                     n_head: int, gate_bias: float = 0.0) -> Tensor:
    """The pairformer's single attention from ``single_attention_`` and the pair-logit norm
    (with its offset) and projection: ``single [N, c_s]`` -> ``single + update``."""
    s = _f64(s)
    single, pair = single.to(F64), pair.to(F64)
    a = _sub(s, "single_attention_")
    x = _ln(single, a, "adaptive_layernorm.layer_norm")
    n, cs = x.shape

    def heads(t: Tensor) -> Tensor:
        return t.reshape(n, n_head, -1).permute(1, 0, 2)

    q, k, v = (heads(_lin(x, a, f"{p}_projection")) for p in ("q", "k", "v"))
    norm, proj = _sub(s, "single_pair_logits_norm"), _sub(s, "single_pair_logits_projection")
    zn = F.layer_norm(pair, pair.shape[-1:], norm["weight"], norm.get("bias"), 1e-5)
    bias = (zn @ proj["weight"].T).permute(2, 0, 1)
    logits = (q * q.shape[-1] ** -0.5) @ k.transpose(-1, -2) + bias
    logits = logits.masked_fill(~token_mask.bool()[None, None, :], -1e9)
    o = (torch.softmax(logits, dim=-1) @ v).permute(1, 0, 2).reshape(n, cs)
    gate = torch.sigmoid(_lin(x, a, "gating_query") + gate_bias)
    return single + F.linear(gate * o, a["adaptive_zero_init.transition2.weight"])


def pairformer_block(z: Tensor, token_mask: Tensor, state: State, *, n_head_pair: int,
                     single: Tensor | None = None, n_head_single: int = 16) -> Tensor | tuple[Tensor, Tensor]:
    """AF3 order (``legacy/pairformer.py:191-230``) on released keys: ``z [N, N, c]``."""
    pm = token_mask[:, None] & token_mask[None, :]
    z = triangle_multiplication(z, pm, _sub(state, "triangle_multiplication_outgoing"), outgoing=True)
    z = triangle_multiplication(z, pm, _sub(state, "triangle_multiplication_incoming"), outgoing=False)
    z = triangle_attention(z, pm, _sub(state, "pair_attention1"), n_head=n_head_pair, ending=False)
    z = triangle_attention(z, pm, _sub(state, "pair_attention2"), n_head=n_head_pair, ending=True)
    z = transition(z, _sub(state, "pair_transition"))
    if single is None:
        return z
    sub = {k: v.to(F64) for k, v in state.items() if k.startswith("single_")}
    single = single_attention(single, z, token_mask, sub, n_head=n_head_single)
    single = transition(single, _sub(state, "single_transition"))
    return z, single


def msa_block(msa: Tensor, z: Tensor, msa_mask: Tensor, token_mask: Tensor, state: State, *,
              n_head_pair: int, n_head_msa: int = 8) -> tuple[Tensor, Tensor]:
    """The AF3 MSA-stack block on released keys (outer product mean, MSA attention, MSA
    transition, then the pair track): ``msa [S, N, c_m]``, ``z [N, N, c_z]``."""
    pm = token_mask[:, None] & token_mask[None, :]
    z = z.to(F64) + outer_product_mean(msa, msa_mask, _sub(state, "outer_product_mean"))
    msa = msa_attention(msa, msa_mask, z, _sub(state, "msa_attention1"), n_head=n_head_msa)
    msa = transition(msa, _sub(state, "msa_transition"))
    z = triangle_multiplication(z, pm, _sub(state, "triangle_multiplication_outgoing"), outgoing=True)
    z = triangle_multiplication(z, pm, _sub(state, "triangle_multiplication_incoming"), outgoing=False)
    if any(k.startswith("pair_attention1.") for k in state):
        z = triangle_attention(z, pm, _sub(state, "pair_attention1"), n_head=n_head_pair, ending=False)
        z = triangle_attention(z, pm, _sub(state, "pair_attention2"), n_head=n_head_pair, ending=True)
    z = transition(z, _sub(state, "pair_transition"))
    return msa, z
