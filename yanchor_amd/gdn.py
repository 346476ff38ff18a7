"""Gated DeltaNet kernels behind the reference's call signatures.

``recurrent_gated_delta_rule`` is the drop-in for the function the GDN layer
binds as ``module.recurrent_gated_delta_rule`` (reference modeling_yanchor.py:
401-407; called at transformers wheel models/qwen3_5/modeling_qwen3_5.py:
508-517 and runtime/model/inference_kernels.py:716).  Like the reference's
in-place FLA launch (runtime/model/inference_kernels.py:147-173) it updates
``initial_state`` in place and returns that same tensor, so the cache's alias
check (modeling_yanchor.py:702-710) skips the copy.
"""
from __future__ import annotations

import torch

from . import _native as N


def _contig(x: torch.Tensor) -> torch.Tensor:
    return x if x.is_contiguous() else x.contiguous()


def recurrent_gated_delta_rule(query, key, value, g=None, beta=None, initial_state=None,
                               output_final_state=True, use_qk_l2norm_in_kernel=True,
                               scale=None, state_indices=None, inplace=True, **unused):
    """Token-recurrent gated delta rule on the GPU.

    query, key ``[B, T, H, K]``; value ``[B, T, HV, V]``; g, beta ``[B, T, HV]``;
    initial_state float32 ``[N, HV, K, V]`` (N >= B, or any N with
    ``state_indices``).  ``state_indices`` (int ``[B]``, -1 = skip) selects the
    state row of each batch row, the slot indirection of the vLLM/SGLang
    adapters.  Returns ``(o [B, T, HV, V], state)``; ``state`` is
    ``initial_state`` itself (updated in place) unless ``inplace=False``, or a
    new zero-initialised tensor when ``initial_state`` is None.  With
    ``output_final_state=False`` the second element is None.
    """
    if g is None or beta is None:
        raise ValueError("recurrent_gated_delta_rule needs g and beta")
    if query.ndim != 4 or key.shape != query.shape or value.ndim != 4:
        raise ValueError("query/key must be [B, T, H, K] and value [B, T, HV, V]")
    b, t, h, kd = key.shape
    hv, vd = value.shape[2], value.shape[3]
    if value.shape[:2] != (b, t) or g.shape != (b, t, hv) or beta.shape != (b, t, hv):
        raise ValueError("value/g/beta shapes do not match query/key")
    if query.dtype != key.dtype or value.dtype != key.dtype:
        raise ValueError("query, key and value must share one dtype")
    dev = N.require_device(query, key, value, g, beta, initial_state, state_indices)
    if initial_state is None:
        if state_indices is not None:
            raise ValueError("state_indices needs an initial_state pool")
        state = torch.zeros(b, hv, kd, vd, device=dev, dtype=torch.float32)
    else:
        if initial_state.dtype != torch.float32:
            raise ValueError("the recurrent state must be float32")
        if initial_state.ndim != 4 or tuple(initial_state.shape[1:]) != (hv, kd, vd):
            raise ValueError(f"initial_state must be [N, {hv}, {kd}, {vd}]")
        if not initial_state.is_contiguous():
            raise ValueError("initial_state must be contiguous (it is updated in place)")
        state = initial_state if inplace else initial_state.clone()
    idx = None
    if state_indices is not None:
        if state_indices.shape != (b,):
            raise ValueError("state_indices must be [B]")
        idx = _contig(state_indices.to(torch.int32))
    elif state.shape[0] < b:
        raise ValueError("state pool has fewer rows than the batch")
    q, k, v, g_, be = (_contig(x) for x in (query, key, value, g, beta))
    o = torch.empty(b, t, hv, vd, device=dev, dtype=value.dtype)
    sc = float(kd ** -0.5 if scale is None else scale)
    N.call("yh_gdn_recurrent", q.data_ptr(), k.data_ptr(), v.data_ptr(), g_.data_ptr(),
           be.data_ptr(), state.data_ptr(), N.ptr(idx), o.data_ptr(), b, t, h, hv, kd, vd,
           state.shape[0], sc, int(bool(use_qk_l2norm_in_kernel)), N.code(q), N.code(g_),
           N.code(be), N.stream_of(q))
    return o, (state if output_final_state else None)


def fused_recurrent_gated_delta_rule(q, k, v, g=None, beta=None, scale=None, initial_state=None,
                                     output_final_state=False, use_qk_l2norm_in_kernel=False,
                                     **kw):
    """FLA-style keyword order (fla.ops.gated_delta_rule.fused_recurrent), the
    name the reference binds at modeling_yanchor.py:404."""
    return recurrent_gated_delta_rule(q, k, v, g=g, beta=beta, initial_state=initial_state,
                                      output_final_state=output_final_state,
                                      use_qk_l2norm_in_kernel=use_qk_l2norm_in_kernel,
                                      scale=scale, inplace=bool(output_final_state), **kw)


def _packed_or_batched(query, key, value, g, beta, cu_seqlens):
    if cu_seqlens is None:
        return None
    if query.shape[0] != 1:
        raise ValueError("with cu_seqlens the inputs must be packed as [1, total, ...]")
    cu = cu_seqlens.to(device=query.device, dtype=torch.int32).contiguous()
    if cu.ndim != 1 or cu.numel() < 1:
        raise ValueError("cu_seqlens must be a 1-D offset vector")
    return cu


def _chunk_kernel_fits(query, value):
    """The MFMA chunk kernels take K = 128, V in {64, 128} and bf16 q/k/v."""
    return (query.ndim == 4 and value.ndim == 4 and query.shape[-1] == 128 and value.shape[-1] in (64, 128)
            and query.dtype == torch.bfloat16)


def chunk_gated_delta_rule(query, key, value, g=None, beta=None, scale=None, initial_state=None,
                           output_final_state=False, use_qk_l2norm_in_kernel=False, cu_seqlens=None,
                           lengths=None, force_recurrent=False, **unused):
    """Prefill form of the gated delta rule with the FLA / Transformers
    signature (bound at modeling_yanchor.py:397, 403; called at transformers
    wheel models/qwen3_5/modeling_qwen3_5.py:519-529).

    Batched: query/key ``[B, T, H, K]``, value ``[B, T, HV, V]``, g/beta
    ``[B, T, HV]``, initial_state ``[B, HV, K, V]``.  Packed varlen:
    ``cu_seqlens`` (int, N + 1 offsets) with inputs ``[1, total, ...]`` and
    initial_state ``[N, HV, K, V]``.  ``initial_state`` is read, not modified;
    returns ``(o, final_state or None)``.

    Inputs with K = 128, V in {64, 128} and bf16 q/k/v run the MFMA chunk
    kernel (chunk 64): packed ones as given, batched ones (the reference's
    own call, T > 1) as B packed sequences of T tokens.  Other shapes, or
    ``force_recurrent=True``, run the token-recurrent kernel over each
    sequence.  ``lengths`` (host ints, one per sequence) lets the chunk
    kernel start the longest sequences first.  The chunk kernel needs no
    scratch memory, so concurrent calls on different streams are independent.
    """
    if g is None or beta is None:
        raise ValueError("chunk_gated_delta_rule needs g and beta")
    cu = _packed_or_batched(query, key, value, g, beta, cu_seqlens)
    if cu is None and _chunk_kernel_fits(query, value) and query.shape[1] > 1 and not force_recurrent:
        # The reference's own call is batched ([B, T, ...], no cu_seqlens):
        # B sequences of T tokens are B * T packed tokens at offsets i * T.
        b, t = query.shape[:2]
        cu_b = torch.arange(0, (b + 1) * t, t, dtype=torch.int32, device=query.device)
        o, st = chunk_gated_delta_rule(
            query.reshape(1, b * t, *query.shape[2:]), key.reshape(1, b * t, *key.shape[2:]),
            value.reshape(1, b * t, *value.shape[2:]), g=g.reshape(1, b * t, -1), beta=beta.reshape(1, b * t, -1),
            scale=scale, initial_state=initial_state, output_final_state=output_final_state,
            use_qk_l2norm_in_kernel=use_qk_l2norm_in_kernel, cu_seqlens=cu_b)
        return o.view(b, t, *o.shape[2:]), st
    if cu is None:
        o, st = recurrent_gated_delta_rule(query, key, value, g=g, beta=beta, initial_state=initial_state,
                                           output_final_state=True,
                                           use_qk_l2norm_in_kernel=use_qk_l2norm_in_kernel, scale=scale,
                                           inplace=False)
        return o, (st if output_final_state else None)
    if query.ndim != 4 or key.shape != query.shape or value.ndim != 4:
        raise ValueError("query/key must be [1, total, H, K] and value [1, total, HV, V]")
    _, total, h, kd = key.shape
    hv, vd = value.shape[2], value.shape[3]
    n = cu.numel() - 1
    if g.shape != (1, total, hv) or beta.shape != (1, total, hv) or value.shape[1] != total:
        raise ValueError("value/g/beta shapes do not match the packed query/key")
    if query.dtype != key.dtype or value.dtype != key.dtype:
        raise ValueError("query, key and value must share one dtype")
    dev = N.require_device(query, key, value, g, beta, initial_state)
    if initial_state is not None and (initial_state.shape != (n, hv, kd, vd)
                                      or initial_state.dtype != torch.float32):
        raise ValueError(f"initial_state must be float32 [{n}, {hv}, {kd}, {vd}]")
    q, k, v, g_, be = (_contig(x) for x in (query, key, value, g, beta))
    o = torch.empty(1, total, hv, vd, device=dev, dtype=value.dtype)
    sc = float(kd ** -0.5 if scale is None else scale)
    if _chunk_kernel_fits(q, v) and not force_recurrent:
        h0 = None if initial_state is None else initial_state.contiguous()
        state = torch.empty(n, hv, kd, vd, device=dev, dtype=torch.float32)
        order = None
        if lengths is not None:  # longest sequences first balances the grid
            order = torch.tensor(sorted(range(n), key=lambda i: -int(lengths[i])), dtype=torch.int32,
                                 device=dev)
        N.call("yh_gdn_chunk_varlen", q.data_ptr(), k.data_ptr(), v.data_ptr(), g_.data_ptr(), be.data_ptr(),
               N.ptr(h0), state.data_ptr(), o.data_ptr(), cu.data_ptr(), N.ptr(order), n, total, h, hv, kd, vd, sc,
               int(bool(use_qk_l2norm_in_kernel)), N.code(q), N.code(g_), N.code(be), None, 0, N.stream_of(q))
        return o, (state if output_final_state else None)
    if initial_state is None:
        state = torch.zeros(n, hv, kd, vd, device=dev, dtype=torch.float32)
    else:
        state = initial_state.clone()
    N.call("yh_gdn_recurrent_varlen", q.data_ptr(), k.data_ptr(), v.data_ptr(), g_.data_ptr(), be.data_ptr(),
           state.data_ptr(), None, cu.data_ptr(), o.data_ptr(), n, h, hv, kd, vd, n, sc,
           int(bool(use_qk_l2norm_in_kernel)), N.code(q), N.code(g_), N.code(be), N.stream_of(q))
    return o, (state if output_final_state else None)
