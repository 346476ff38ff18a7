"""Decode-layer glue around the hot path, on the CPU (oracle; test
infrastructure only).

Restates, with the reference's own dtypes and rounding points (bf16 inputs
round where the reference's bf16 torch ops round; float64 inputs give the
exact function):

* ``rms_norm``              Qwen3_5RMSNorm (wheel
                            transformers/models/qwen3_5/modeling_qwen3_5.py:720-734):
                            x / rms(x) * (1 + w) in fp32, cast back.
* ``gated_rms_norm``        Qwen3_5RMSNormGated (wheel:175-190): norm in fp32,
                            cast, times w in the weight dtype, times
                            silu(gate) in fp32, cast.
* ``causal_conv1d_update``  torch_causal_conv1d_update (wheel:210-225) with the
                            SiLU activation: [state | x] in the weight dtype,
                            depthwise conv1d (output in that dtype), SiLU,
                            state <- last state_len columns.
* ``causal_conv1d_update_cuda``  the CUDA backend's decode conv update
                            (causal-conv1d==1.6.2.post1, bound at
                            modeling_yanchor.py:392-405): fp32 sum and SiLU,
                            one rounding; restated from the package's
                            published kernel (the package is absent).
* ``gdn_gates``             _qwen35_fused_gdn_gates_kernel
                            (runtime/model/inference_kernels.py:668-691):
                            beta = sigmoid(b) stored in b's dtype, decay
                            g = -exp(A_log) * softplus(a + dt_bias) in fp32
                            with the softplus threshold 20.
* ``rotate_half``,          rotate_half (wheel:545-549) and _memory_rope
  ``memory_rope``           (modeling_yanchor.py:46-49): rotate-half RoPE on
                            the first cos.shape[-1] dims, in the operands'
                            dtype.
* ``query_scores``          IndependentGQAMemory._query_scores
                            (modeling_yanchor.py:168-176): q_norm(q_proj u),
                            read gate tanh(read_scale) * 2 * sigmoid(<q, w> /
                            sqrt(D) + b) before RoPE, RoPE, admission scores
                            silu(admission_down u) . admission_up^T in fp32.
* ``write_kv``              IndependentGQAMemory._write_kv (modeling_yanchor.py:
                            147-166): z = u + down(silu(gate u) * up u);
                            key = RoPE(k_norm(k_proj z)); value = v_proj z.
* ``ring_decode_attention`` fixed_memory_physical_ring_decode_attention
                            (runtime/model/inference_kernels.py:1881-1898):
                            softmax(q K^T / sqrt(D)) V over the live ring
                            slots, query heads grouped on the ring's KV heads,
                            then ``* sigmoid(gate)`` (Qwen3_5FixedWindowAttention
                            forward, modeling_yanchor.py:871-875; the fused
                            form inference_kernels.py:1899-1915 rounds
                            sigmoid(gate) to bf16 before the product).
* ``ring_write``            the chronological ring write
                            (runtime/model/inference_kernels.py:1828-1856):
                            one token's key, value and validity into ring slot
                            ``index``.

Pins (tests/test_oracle_glue.py): RMSNorm against torch's F.rms_norm; the
gated norm against F.rms_norm times F.silu; the conv update fed token by
token against F.conv1d over the whole causal sequence, and in bf16 against
F.conv1d in bf16; the CUDA-backend conv update against the torch form
in float64 (equal) and in bf16 (within the conv-output rounding); the gates against F.softplus (threshold 20) and
torch.sigmoid, and the closed form at a = 0; RoPE against the complex
product (x1 + i x2) e^{i theta} and the identity at position 0; the read gate
at read_scale = 0 (zero) and its bound 2 tanh(read_scale); write_kv with a
zero down projection (the reference's initialisation) reduces to
RoPE(k_norm(k_proj u)); the ring read against F.scaled_dot_product_attention
with the boolean mask and enable_gqa (the reference's own call), plus the
closed forms for one live slot and for equal keys.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def _compute_dtype(x: torch.Tensor) -> torch.dtype:
    """Where the reference upcasts to float32, float64 inputs stay float64."""
    return torch.float64 if x.dtype == torch.float64 else torch.float32


def rms_norm(x, weight, eps=1e-6):
    """Qwen3_5RMSNorm (wheel:720-734): (x / sqrt(mean(x^2) + eps)) * (1 + w),
    computed in fp32 and cast back to x's dtype."""
    ct = _compute_dtype(x)
    xf = x.to(ct)
    out = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (out * (1.0 + weight.to(ct))).to(x.dtype)


def gated_rms_norm(x, gate, weight, eps=1e-6):
    """Qwen3_5RMSNormGated (wheel:175-190): normalise in fp32, cast to the
    input dtype, multiply by the weight (in the weight / input dtype), then
    by silu(gate) in fp32, cast to the input dtype."""
    ct = _compute_dtype(x)
    h = x.to(ct)
    h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    h = weight * h.to(x.dtype)
    h = h * F.silu(gate.to(ct))
    return h.to(x.dtype)


def causal_conv1d_update(x, conv_state, weight, bias=None):
    """torch_causal_conv1d_update with SiLU (wheel:210-225).

    x [B, C, T] (new inputs), conv_state [B, C, S] (the last S inputs, oldest
    first; updated in place to the last S columns of [state | x]), weight
    [C, K] with K <= S + 1.  Output [B, C, T] in x's dtype:
    silu(conv1d([state | x].to(w.dtype), w)[..., -T:]), the conv output and the
    activation each rounded to the weight dtype.
    """
    t = x.shape[-1]
    s = conv_state.shape[-1]
    full = torch.cat([conv_state, x], dim=-1).to(weight.dtype)
    conv_state.copy_(full[:, :, -s:])
    k = weight.shape[-1]
    ct = _compute_dtype(weight)
    windows = full.to(ct).unfold(-1, k, 1)                        # [B, C, S + T - K + 1, K]
    out = (windows * weight.to(ct)[None, :, None, :]).sum(-1)
    if bias is not None:
        out = out + bias.to(ct)[None, :, None]
    out = out.to(weight.dtype)                                     # conv1d output dtype
    out = F.silu(out.to(ct)).to(weight.dtype)                     # F.silu on that tensor
    return out[:, :, -t:].to(x.dtype)


def causal_conv1d_update_cuda(x, conv_state, weight, bias=None):
    """The decode conv update the reference's CUDA backend binds
    (modeling_yanchor.py:392-405: ``causal_conv1d_update`` of the third-party
    package causal-conv1d==1.6.2.post1, requirements.txt:25; not in the
    reference tree and not installed here).  Restated from that package's
    published update kernel: the window and weights are widened to fp32, the
    depthwise sum (plus bias) and the SiLU are evaluated in fp32, and the
    result is written once in x's dtype; the state shifts as in
    ``causal_conv1d_update``.  Same layouts as ``causal_conv1d_update``.
    Parity of the package itself is unpinned (it is absent); this function is
    pinned by equalling ``causal_conv1d_update`` in float64, where neither
    rounds, and by differing from it in bf16 by at most the rounding of the
    conv output before the SiLU."""
    t = x.shape[-1]
    s = conv_state.shape[-1]
    full = torch.cat([conv_state, x.to(conv_state.dtype)], dim=-1)
    conv_state.copy_(full[:, :, -s:])
    k = weight.shape[-1]
    ct = _compute_dtype(x)
    windows = full.to(ct).unfold(-1, k, 1)
    out = (windows * weight.to(ct)[None, :, None, :]).sum(-1)
    if bias is not None:
        out = out + bias.to(ct)[None, :, None]
    return F.silu(out)[:, :, -t:].to(x.dtype)


def gdn_gates(b, a, a_log, dt_bias):
    """_qwen35_fused_gdn_gates_kernel (inference_kernels.py:668-691):
    beta = 1 / (1 + exp(-b)) in fp32, stored in b's dtype; decay
    g = -exp(A_log) * softplus(a + dt_bias) in fp32, softplus = identity above
    20.  Returns (beta, g)."""
    ct = _compute_dtype(b)
    bf, af = b.to(ct), a.to(ct)
    x = af + dt_bias.to(ct)
    sp = torch.where(x > 20.0, x, torch.log1p(torch.exp(torch.clamp(x, max=20.0))))
    beta = (1.0 / (1.0 + torch.exp(-bf))).to(b.dtype)
    return beta, -torch.exp(a_log.to(ct)) * sp


def rotate_half(x):
    """rotate_half (wheel:545-549): [-x2, x1] of the halves of the last dim."""
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def memory_rope(values, cos, sin):
    """_memory_rope (modeling_yanchor.py:46-49): rotate-half RoPE of the first
    cos.shape[-1] dims, the rest passed through; in the operands' dtype."""
    width = cos.shape[-1]
    rotated = values[..., :width]
    return torch.cat((rotated * cos + rotate_half(rotated) * sin, values[..., width:]), -1)


def rope_cos_sin(positions, inv_freq, dtype):
    """cos / sin [..., 2 * len(inv_freq)] of the rotate-half layout, computed
    in fp32 and cast to ``dtype`` as the text rotary embedding returns them
    (for text positions every mrope section carries the same position)."""
    ang = positions.to(torch.float32)[..., None] * inv_freq.to(torch.float32)
    ang = torch.cat((ang, ang), -1)
    return ang.cos().to(dtype), ang.sin().to(dtype)


def query_read_gate(query_normed, read_scale, gate_weight, gate_bias):
    """The read gate of _query_scores (modeling_yanchor.py:170), taken from
    the normed, not yet rotated query [..., H, D]:
    tanh(read_scale) * 2 * sigmoid(sum(q * w, -1) / sqrt(D) + b), in the
    parameters' / query's dtype as torch evaluates it."""
    d = query_normed.shape[-1]
    return read_scale.tanh() * 2 * torch.sigmoid((query_normed * gate_weight).sum(-1) / math.sqrt(d) + gate_bias)


def admission_scores(features_pre, admission_up):
    """Admission scores of _query_scores (modeling_yanchor.py:173-175): silu
    of the admission_down output (in its dtype), then a float32 product with
    admission_up (autocast off)."""
    return F.linear(F.silu(features_pre).float(), admission_up.float())


def query_scores(u, q_proj, q_norm_w, read_scale, gate_weight, gate_bias, admission_down, admission_up, cos, sin,
                 heads, eps=1e-6):
    """IndependentGQAMemory._query_scores (modeling_yanchor.py:168-176) for u
    [..., hidden]: returns (query [..., H, D] rotated, scores [..., G] fp32,
    gate [..., H]).  cos / sin [..., rotary] broadcast over heads."""
    q = F.linear(u, q_proj).unflatten(-1, (heads, -1))
    q = rms_norm(q, q_norm_w, eps)
    gate = query_read_gate(q, read_scale, gate_weight, gate_bias)
    q = memory_rope(q, cos[..., None, :], sin[..., None, :])
    return q, admission_scores(F.linear(u, admission_down), admission_up), gate


def silu_mul(gate, up):
    """silu(gate) * up in the operands' dtype (modeling_yanchor.py:166; the
    fused form inference_kernels.py:642-655 rounds silu(gate) to bf16 first,
    which is what torch's bf16 F.silu does)."""
    return F.silu(gate) * up


def write_kv(u, write_gate, write_up, write_down, k_proj, v_proj, k_norm_w, cos, sin, groups, eps=1e-6):
    """IndependentGQAMemory._write_kv (modeling_yanchor.py:147-166): returns
    (key [..., G, D] normed and rotated, value [..., G, D])."""
    z = u + F.linear(silu_mul(F.linear(u, write_gate), F.linear(u, write_up)), write_down)
    key = rms_norm(F.linear(z, k_proj).unflatten(-1, (groups, -1)), k_norm_w, eps)
    value = F.linear(z, v_proj).unflatten(-1, (groups, -1)).contiguous()
    return memory_rope(key, cos[..., None, :], sin[..., None, :]), value


def ring_decode_attention(query, ring_key, ring_value, valid, gate=None):
    """fixed_memory_physical_ring_decode_attention (inference_kernels.py:
    1881-1898) and the output gate.

    query [B, 1, H, D]; ring_key / ring_value [B, G, W, D] with H a multiple of
    G (query head h reads KV head h // (H / G)); valid [B, W] (or [B, G, W])
    bool.  softmax(q k / sqrt(D)) over the valid slots, accumulated in fp32
    (float64 for float64 inputs), output in the query dtype; with ``gate``
    [B, H, D]: output * sigmoid(gate), sigmoid rounded to the query dtype.
    A row with no valid slot gives 0 (the reference never reads one: the
    decode token is written before the read).
    """
    b, _, h, d = query.shape
    g = ring_key.shape[1]
    ct = _compute_dtype(query)
    mask = valid if valid.ndim == 3 else valid[:, None, :].expand(b, g, valid.shape[-1])
    q = query[:, 0].to(ct).reshape(b, g, h // g, d)
    logits = torch.einsum("bgrd,bgwd->bgrw", q, ring_key.to(ct)) / math.sqrt(d)
    logits = logits.masked_fill(~mask[:, :, None, :], -math.inf)
    m = logits.amax(-1, keepdim=True)
    p = torch.where(mask[:, :, None, :], torch.exp(logits - torch.where(torch.isfinite(m), m, 0)), 0)
    den = p.sum(-1, keepdim=True)
    out = torch.einsum("bgrw,bgwd->bgrd", p, ring_value.to(ct)) / torch.where(den > 0, den, 1)
    out = out.reshape(b, 1, h, d).to(query.dtype)
    if gate is not None:
        out = out * torch.sigmoid(gate.to(ct)).to(query.dtype)[:, None]
    return out


def ring_write(ring_key, ring_value, ring_valid, key, value, valid, index):
    """The chronological ring write (inference_kernels.py:1828-1856): one
    token's key / value [B, G, D] and validity [B] into slot ``index`` ([B]
    ints, or one int) of ring_key / ring_value [B, G, W, D] and ring_valid
    [B, W]; in place."""
    rows = torch.arange(key.shape[0])
    idx = torch.as_tensor(index).expand(key.shape[0])
    ring_key[rows, :, idx] = key
    ring_value[rows, :, idx] = value
    ring_valid[rows, idx] = valid


def causal_conv1d_prefill(x, window, weight):
    """The GDN layer's causal conv1d + SiLU over a prompt piece that
    continues ``window`` (the causal-conv1d prefill call of the CUDA backend,
    modeling_yanchor.py:392-407, with the previous inputs as the initial
    state), in the CUDA form: taps widened to fp32 (float64 for float64
    inputs), sum and SiLU there, one rounding to x's dtype.

    x [T, C] the piece's inputs; window [S, C] the S inputs before it, oldest
    first (zeros for a fresh sequence); weight [C, S + 1].  Returns (y [T, C],
    the new window: the last S rows of [window | x]).  Pinned against
    ``causal_conv1d_update_cuda`` fed one token at a time, and, from a zero
    window in float64, against F.conv1d over the causally padded sequence."""
    t, s = x.shape[0], window.shape[0]
    ct = _compute_dtype(x)
    full = torch.cat([window.to(x.dtype), x], 0)                    # [S + T, C]
    k = weight.shape[-1]
    if t == 0:
        return x.clone(), full[full.shape[0] - s:].clone()
    fc, wc = full.to(ct).contiguous(), weight.to(ct).t().contiguous()    # wc[j]: tap j of every channel
    y = fc[0:t] * wc[0]
    for j in range(1, k):                                            # the K taps, oldest first
        y = y + fc[j: j + t] * wc[j]
    return F.silu(y).to(x.dtype), full[full.shape[0] - s:].clone()


def swa_prefill_attention(query, key, value, window, *, query_start=0, key_valid=None):
    """reference_swa (modeling_yanchor.py:412-427): query [B, L, H, D] at
    positions query_start .. query_start + L - 1 over key / value [B, S, G, D]
    at positions 0 .. S - 1, each query reading the keys in
    [p - window + 1, p] (and ``key_valid`` [B, S] if given), query heads
    grouped on the KV heads (enable_gqa), fp32 accumulation (float64 for
    float64 inputs), output in the query dtype.  flash_swa (429-449, the CUDA
    path's flash_attn call with causal=True and window_size=(window - 1, 0))
    computes the same function.  Pinned against F.scaled_dot_product_attention
    with is_causal (window >= S), the token-by-token ring read
    (``ring_decode_attention`` after each ``ring_write``), and window = 1
    (each query returns its own value)."""
    b, l, h, d = query.shape
    s, g = key.shape[1], key.shape[2]
    ct = _compute_dtype(query)
    qpos = torch.arange(l) + int(query_start)
    kpos = torch.arange(s)
    allowed = (kpos[None] <= qpos[:, None]) & (kpos[None] >= qpos[:, None] - int(window) + 1)   # [L, S]
    allowed = allowed[None, None].expand(b, g, l, s)
    if key_valid is not None:
        allowed = allowed & key_valid[:, None, None, :].bool()
    q = query.to(ct).reshape(b, l, g, h // g, d).permute(0, 2, 3, 1, 4)        # [B, G, R, L, D]
    logits = torch.einsum("bgrld,bgsd->bgrls", q, key.to(ct).transpose(1, 2)) / math.sqrt(d)
    logits = logits.masked_fill(~allowed[:, :, None], -math.inf)
    m = logits.amax(-1, keepdim=True)
    p = torch.exp(logits - torch.where(torch.isfinite(m), m, 0))
    den = p.sum(-1, keepdim=True)
    out = torch.einsum("bgrls,bgsd->bgrld", p, value.to(ct).transpose(1, 2)) / torch.where(den > 0, den, 1)
    return out.permute(0, 3, 1, 2, 4).reshape(b, l, h, d).to(query.dtype)
