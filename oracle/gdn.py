"""Gated delta rule on the CPU (oracle; test infrastructure only).

Restates the arithmetic of the vendored Transformers Qwen3.5 GDN reference
(``wheels/transformers-5.7.0.dev0-py3-none-any.whl``, file
``transformers/models/qwen3_5/modeling_qwen3_5.py``, cited below as ``wheel:``):

* ``l2norm``                      wheel:228-231
* ``recurrent_gated_delta_rule``  wheel:314-353 (torch_recurrent_gated_delta_rule)
* ``chunk_gated_delta_rule``      wheel:234-311 (torch_chunk_gated_delta_rule)
* varlen packing                  cu_seqlens form of the FLA call mirrored at
                                  runtime/model/inference_kernels.py:147
* ``gdn_gates``                   runtime/model/inference_kernels.py:668-680 and
                                  wheel:500-502

Layouts (same as the reference callers): q, k ``[B, T, H, K]``; v
``[B, T, HV, V]``; g, beta ``[B, T, HV]``; state ``[B, HV, K, V]`` (the value
dimension is contiguous).  Value head ``j`` reads key head ``j // (HV // H)``,
which is what ``repeat_interleave(HV // H, dim=2)`` of q/k does at
runtime/model/inference_kernels.py:712-715.

Pins (tests/test_oracle_gdn.py): closed forms for T=1 from a zero state and for
beta=0; the delta-rule overwrite invariant; chunked == recurrent for chunk sizes
16/32/64; packed varlen == per-sequence runs == left-padded batch.
"""
from __future__ import annotations

import torch


def l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """x / sqrt(sum(x^2) + eps) over the last dim (wheel:228-231: eps inside rsqrt)."""
    return x * torch.rsqrt((x * x).sum(dim=-1, keepdim=True) + eps)


def _expand_heads(x: torch.Tensor, hv: int) -> torch.Tensor:
    h = x.shape[2]
    if hv % h:
        raise ValueError("value heads must be a multiple of key heads")
    return x if h == hv else x.repeat_interleave(hv // h, dim=2)


def recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=None, *, use_qk_l2norm=True,
                               scale=None, dtype=torch.float64):
    """Token-by-token gated delta rule (wheel:314-353).

    Per step t, per (batch, value head):
        S <- exp(g_t) * S
        kv = S^T k_t                      (sum over the key dim)
        delta = beta_t * (v_t - kv)
        S <- S + k_t delta^T
        o_t = S^T (q_t * scale)
    with q, k L2-normalised first when ``use_qk_l2norm`` (wheel:336-338) and
    scale = K ** -0.5 applied after the normalisation (wheel:345-346).

    Returns (o [B, T, HV, V], final_state [B, HV, K, V]) in ``dtype``.
    """
    hv = v.shape[2]
    q, k = (_expand_heads(x, hv).to(dtype) for x in (q, k))
    v, g, beta = (x.to(dtype) for x in (v, g, beta))
    if use_qk_l2norm:
        q, k = l2norm(q), l2norm(k)
    b, t, _, kd = k.shape
    vd = v.shape[-1]
    q = q * (kd ** -0.5 if scale is None else scale)
    state = (torch.zeros(b, hv, kd, vd, dtype=dtype) if initial_state is None
             else initial_state.to(dtype))
    out = torch.zeros(b, t, hv, vd, dtype=dtype)
    for i in range(t):
        state = state * g[:, i].exp()[..., None, None]
        kt = k[:, i]                                   # [B, HV, K]
        kv = torch.einsum("bhkv,bhk->bhv", state, kt)
        delta = beta[:, i][..., None] * (v[:, i] - kv)
        state = state + kt[..., :, None] * delta[..., None, :]
        out[:, i] = torch.einsum("bhkv,bhk->bhv", state, q[:, i])
    return out, state


def chunk_gated_delta_rule(q, k, v, g, beta, initial_state=None, *, chunk_size=64,
                           use_qk_l2norm=True, scale=None, dtype=torch.float64):
    """Chunked (WY / UT-transform) form of the same recurrence (wheel:234-311).

    Within each chunk of C tokens (T padded with zeros to a multiple of C, as
    wheel:255-262 does):
        G   = cumsum(g)                                   (wheel:275)
        D   = tril(exp(tril(G_i - G_j)))                  (wheel:276, tril before exp)
        A   = -(k*beta) k^T * D, strictly lower           (wheel:277)
        A  <- (I - A)^{-1} by row forward substitution, i.e. T = (I + L)^{-1}
                                                          (wheel:278-282)
        U   = A (v*beta);  W = A (k*beta*exp(G))          (wheel:283-284)
    then the inter-chunk scan (wheel:293-304):
        v_new = U - W S
        o     = (q*exp(G)) S + ((q k^T) * D_incl_diag) v_new
        S    <- exp(G_last) S + (k*exp(G_last - G))^T v_new
    """
    hv = v.shape[2]
    q, k = (_expand_heads(x, hv).to(dtype) for x in (q, k))
    v, g, beta = (x.to(dtype) for x in (v, g, beta))
    if use_qk_l2norm:
        q, k = l2norm(q), l2norm(k)
    b, t, _, kd = k.shape
    vd = v.shape[-1]
    c = chunk_size
    pad = (-t) % c
    # [B, HV, T, D] layout for the chunk algebra
    q, k, v = (torch.nn.functional.pad(x.transpose(1, 2), (0, 0, 0, pad)) for x in (q, k, v))
    g, beta = (torch.nn.functional.pad(x.transpose(1, 2), (0, pad)) for x in (g, beta))
    q = q * (kd ** -0.5 if scale is None else scale)
    n = (t + pad) // c
    q, k, v = (x.reshape(b, hv, n, c, x.shape[-1]) for x in (q, k, v))
    g, beta = (x.reshape(b, hv, n, c) for x in (g, beta))
    kb, vb = k * beta[..., None], v * beta[..., None]
    gc = g.cumsum(-1)
    diff = gc[..., :, None] - gc[..., None, :]
    lower = torch.ones(c, c, dtype=torch.bool).tril()
    decay = torch.where(lower, diff, torch.zeros((), dtype=dtype)).exp() * lower
    strict = lower & ~torch.eye(c, dtype=torch.bool)
    a = -(kb @ k.transpose(-1, -2)) * decay * strict
    # forward substitution: row i of T = e_i + sum_{m<i} a[i, m] * T[m]
    tmat = torch.zeros_like(a)
    eye = torch.eye(c, dtype=dtype)
    for i in range(c):
        tmat[..., i, :] = eye[i] + (a[..., i, :i, None] * tmat[..., :i, :]).sum(-2)
    u = tmat @ vb
    w = tmat @ (kb * gc.exp()[..., None])
    state = (torch.zeros(b, hv, kd, vd, dtype=dtype) if initial_state is None
             else initial_state.to(dtype))
    out = torch.zeros(b, hv, n, c, vd, dtype=dtype)
    for j in range(n):
        qj, kj, gj = q[:, :, j], k[:, :, j], gc[:, :, j]
        v_new = u[:, :, j] - w[:, :, j] @ state
        attn = (qj @ kj.transpose(-1, -2)) * decay[:, :, j]
        out[:, :, j] = (qj * gj.exp()[..., None]) @ state + attn @ v_new
        glast = gj[..., -1]
        state = (state * glast.exp()[..., None, None]
                 + (kj * (glast[..., None] - gj).exp()[..., None]).transpose(-1, -2) @ v_new)
    out = out.reshape(b, hv, n * c, vd)[:, :, :t].transpose(1, 2)
    return out, state


def varlen(fn, q, k, v, g, beta, cu_seqlens, initial_state=None, **kw):
    """Packed-sequence form: inputs are ``[1, sum(T), ...]`` and ``cu_seqlens``
    (int, length N+1, exclusive prefix sum of lengths) delimits N independent
    sequences; ``initial_state`` is ``[N, HV, K, V]`` or None (zeros).  Returns
    (o [1, sum(T), HV, V], final states [N, HV, K, V]).  Same contract as the
    ``cu_seqlens`` argument of the FLA call at
    runtime/model/inference_kernels.py:147.
    """
    cu = [int(x) for x in cu_seqlens]
    outs, finals = [], []
    for i in range(len(cu) - 1):
        s, e = cu[i], cu[i + 1]
        h0 = None if initial_state is None else initial_state[i:i + 1]
        o, st = fn(q[:, s:e], k[:, s:e], v[:, s:e], g[:, s:e], beta[:, s:e], h0, **kw)
        outs.append(o)
        finals.append(st)
    return torch.cat(outs, 1), torch.cat(finals, 0)


def gdn_gates(b, a, a_log, dt_bias, dtype=torch.float64):
    """beta = sigmoid(b); g = -exp(A_log) * softplus(a + dt_bias), softplus
    threshold 20 (runtime/model/inference_kernels.py:668-680; wheel:500-502)."""
    b, a, a_log, dt_bias = (x.to(dtype) for x in (b, a, a_log, dt_bias))
    x = a + dt_bias
    sp = torch.where(x > 20.0, x, torch.log1p(torch.exp(torch.clamp(x, max=20.0))))
    return torch.sigmoid(b), -torch.exp(a_log) * sp
