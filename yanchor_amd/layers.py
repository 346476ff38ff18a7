"""Fused decode-layer neighbours of the hot path (HIP kernels, bf16 activations).

RMSNorm with a fused residual add, the GDN decode prologue (causal conv1d
update + SiLU + q/k/v split + beta/g gates), the gated RMSNorm of the GDN
output, silu(gate) * up, per-head RMSNorm + partial RoPE, and the skinny
projection of the decode step.  Each keeps the rounding points of the torch
formulation it replaces (cited per function).
"""
from __future__ import annotations

import ctypes

import torch

from . import _native as N


def _bf16(*ts):
    for t in ts:
        if t is not None and t.dtype != torch.bfloat16:
            raise ValueError("fused layer kernels take bfloat16 activations")


# Normed decode rows (at most 128, the batch of a decode step) are the x of
# the packed projections that follow, and are written 256 elements longer
# than their width (the tensor returned is a view of the first D columns).
# Measured on MI355X at K = 2560 with an x that stays in L2 (HIP graphs over
# rotating weights): x rows 5120 bytes apart cost gate/up 31.2 us and the GDN
# input 29.7 us, rows 5632 bytes apart 27.8 and 25.6 us (every stride from
# 5504 bytes up gave the same; K = 4096 and 9728 were indifferent).  In the
# decode step, where each x is freshly written by the norm, the 96-column
# projections gained 0.4 us a call (29.5 -> 29.1 us) and the step 0.3 %.
_ROW_PAD = 256


def _normed_rows(m, d, dtype, device):
    if m <= 256 and d % 8 == 0:
        return torch.empty(m, d + _ROW_PAD, dtype=dtype, device=device)[:, :d]
    return torch.empty(m, d, dtype=dtype, device=device)


def rmsnorm(x, w, eps, residual=None, plus_one=True, w2=None, w2_row=None):
    """Qwen3.5 RMSNorm over the last dim (x / rms(x) * (1 + w)).  With
    ``residual``: s = x + residual is formed first and ``(norm(s), s)`` is
    returned (the fused residual RMSNorm, runtime/model/inference_kernels.py:
    1767-1797).  ``w2``: the same row normed with a second weight is appended
    to the result (one launch when x is split-K partials); with ``w2_row`` (>=
    D, x split-K partials) it is the first D columns of rows ``w2_row`` wide,
    the rest left for the caller."""
    if isinstance(x, Partials):
        return _rmsnorm_partials(x, w, eps, residual, plus_one, w2, w2_row)
    if w2 is not None:
        first = rmsnorm(x, w, eps, residual, plus_one)
        if residual is None:
            return first, rmsnorm(x, w2, eps, None, plus_one)
        return first + (rmsnorm(first[1], w2, eps, None, plus_one),)
    _bf16(x, w, residual)
    d = x.shape[-1]
    if x.stride(-1) != 1 or (x.ndim > 1 and x.stride(-2) % 8):
        x = x.contiguous()
    rows = x.numel() // d
    N.require_device(x, w, residual)
    out = _normed_rows(rows, d, x.dtype, x.device) if x.ndim == 2 else torch.empty(x.shape, dtype=x.dtype,
                                                                                       device=x.device)
    res_out = None
    if residual is not None:
        residual = residual.contiguous()
        res_out = torch.empty_like(residual)
    x_stride = x.stride(-2) if x.ndim > 1 else d
    if x.ndim > 2 and not x.is_contiguous():
        x = x.contiguous()
        x_stride = d
    N.call("yh_rmsnorm", x.data_ptr(), x_stride, N.ptr(residual), N.ptr(res_out), w.data_ptr(), out.data_ptr(),
           out.stride(0) if out.ndim == 2 else d, rows, d, float(eps), int(plus_one), N.stream_of(x))
    return out if residual is None else (out, res_out)


def decode_inputs(tokens, positions, embed, w, inv_freq, eps, *, ring_stride, window, finished=None,
                  slot_rows=None):
    """Inputs of one decode step in one launch: (h = embed[tokens], xn =
    RMSNorm(h) * (1 + w), cos, sin [B, 2 len(inv_freq)] float32 of positions *
    inv_freq (rotate-half layout), ring_rows = arange(B) * ring_stride +
    positions % window, valid = ~finished & (slot_rows >= 0) or None).  The
    embedding lookup and rotary tables of the model forward
    (modeling_yanchor.py:932, 951)."""
    _bf16(embed, w)
    if tokens.dtype != torch.int64 or positions.dtype != torch.int64 or tokens.shape != positions.shape or \
            tokens.ndim != 1:
        raise ValueError("tokens and positions must be int64 [B]")
    tokens, positions = tokens.contiguous(), positions.contiguous()
    if (finished is None) != (slot_rows is None):
        raise ValueError("valid needs both finished and slot_rows")
    if finished is not None and (finished.dtype != torch.bool or slot_rows.dtype != torch.int64 or
                                 finished.shape != tokens.shape or slot_rows.shape != tokens.shape or
                                 not finished.is_contiguous() or not slot_rows.is_contiguous()):
        raise ValueError("finished / slot_rows must be contiguous bool / int64 [B]")
    if inv_freq.dtype != torch.float32 or not inv_freq.is_contiguous() or not embed.is_contiguous():
        raise ValueError("inv_freq must be contiguous float32 and embed contiguous")
    dev = N.require_device(tokens, positions, embed, w, inv_freq, finished, slot_rows)
    b, (v, d), rd = tokens.shape[0], embed.shape, 2 * inv_freq.numel()
    h = torch.empty(b, d, dtype=torch.bfloat16, device=dev)
    xn = torch.empty_like(h)
    cos = torch.empty(b, rd, dtype=torch.float32, device=dev)
    sin = torch.empty_like(cos)
    rows = torch.empty(b, dtype=torch.int64, device=dev)
    valid = None if finished is None else torch.empty(b, dtype=torch.bool, device=dev)
    N.call("yh_decode_inputs", tokens.data_ptr(), positions.data_ptr(), embed.data_ptr(), v, w.data_ptr(),
           inv_freq.data_ptr(), N.ptr(finished), N.ptr(slot_rows), h.data_ptr(), xn.data_ptr(), cos.data_ptr(),
           sin.data_ptr(), rows.data_ptr(), N.ptr(valid), b, d, rd, int(ring_stride), int(window), float(eps),
           N.stream_of(tokens))
    return h, xn, cos, sin, rows, valid


def _rmsnorm_partials(p, w, eps, residual, plus_one, w2=None, w2_row=None):
    r1, part2 = p.residual, None
    if isinstance(r1, Partials):   # a second projection's partials: the residual of the first
        if r1.shape != p.shape or r1.residual is not None:
            raise ValueError("the residual partials must match the projection and carry no residual")
        part2, r1 = r1.part, None
        N.require_device(part2)
    _bf16(w, residual, r1, w2)
    m, d = p.shape
    N.require_device(p.part, w, residual, r1, w2)
    out = _normed_rows(m, d, torch.bfloat16, p.device)
    out2 = None
    if w2 is not None:
        row = d if w2_row is None else int(w2_row)
        if row < d or row % 8:
            raise ValueError("w2_row must be at least D and a multiple of 8")
        out2 = torch.empty(m, row, dtype=torch.bfloat16, device=p.device)[:, :d]
    res_out = None
    if residual is not None:
        residual = residual.contiguous()
        res_out = torch.empty_like(residual)
    if r1 is not None and (r1.stride(-1) != 1 or r1.stride(0) % 8 or r1.data_ptr() % 16):
        r1 = r1.contiguous()
    N.call("yh_rmsnorm_partials", p.part.data_ptr(), p.part.shape[0], N.ptr(r1), 0 if r1 is None else r1.stride(0),
           N.ptr(part2), 0 if part2 is None else part2.shape[0], N.ptr(residual), N.ptr(res_out), w.data_ptr(), out.data_ptr(), out.stride(0), m, d, float(eps),
           int(plus_one), N.ptr(w2), N.ptr(out2), 0 if out2 is None else out2.stride(0), N.stream_of(p.part))
    res = (out,) if residual is None else (out, res_out)
    res = res if out2 is None else res + (out2,)
    return res[0] if len(res) == 1 else res


def gdn_decode_fused(proj, conv_state, conv_w, a_log, dt_bias, state, norm_w, eps, *, heads, head_dim, z_offset,
                     b_offset, a_offset, scale=None, state_indices=None):
    """One decode token of a GDN layer's core, one launch: ``gdn_decode_prep``
    + the gated delta rule (L2-normed q/k, ``state`` [N, H, D, D] float32, or
    float16 as the reference's throughput profile stores it, in place) +
    ``gated_rmsnorm`` of the output, bit for bit.  proj [B, P] bf16
    (qkv | z | b | a), conv_state [B, 3, conv_dim] shifted in place -> y
    [B, H * D] bf16."""
    _bf16(proj, conv_state, conv_w, norm_w)
    b = proj.shape[0]
    h, d = int(heads), int(head_dim)
    conv_dim = 3 * h * d
    if proj.stride(-1) != 1 or conv_state.shape != (b, 3, conv_dim) or not conv_state.is_contiguous():
        raise ValueError("proj must have unit column stride and conv_state be contiguous [B, 3, conv_dim]")
    if state.dtype not in (torch.float32, torch.float16) or not state.is_contiguous() or \
            tuple(state.shape[1:]) != (h, d, d):
        raise ValueError("state must be contiguous float32 or float16 [N, H, D, D]")
    dev = N.require_device(proj, conv_state, conv_w, a_log, dt_bias, state, norm_w, state_indices)
    idx = None if state_indices is None else state_indices.to(torch.int32).contiguous()
    y = torch.empty(b, h * d, dtype=torch.bfloat16, device=dev)
    sc = float(d ** -0.5 if scale is None else scale)
    N.call("yh_gdn_decode_fused", proj.data_ptr(), proj.stride(0), conv_state.data_ptr(), conv_w.contiguous().data_ptr(),
           a_log.float().contiguous().data_ptr(), dt_bias.float().contiguous().data_ptr(), state.data_ptr(),
           N.DTYPE_CODE[state.dtype], N.ptr(idx), norm_w.contiguous().data_ptr(), y.data_ptr(), b, h, h, d, d,
           conv_dim, int(z_offset),
           int(b_offset), int(a_offset), state.shape[0], sc, 1, float(eps), N.stream_of(proj))
    return y


def gdn_decode_prep(proj, conv_state, conv_w, a_log, dt_bias, *, conv_dim, qk_dim, hv, b_offset, a_offset):
    """Decode prologue of a GDN layer from the packed projection ``proj``
    [B, P] (qkv | z | b | a): returns q, k [B, 1, H, dk], v [B, 1, HV, dv]
    (bf16), g, beta [B, 1, HV] (float32); ``conv_state`` [B, 3, conv_dim] is
    shifted in place.  Replaces the graph-safe conv update and the fused GDN
    gates (runtime/model/inference_kernels.py:339-376, 668-691)."""
    _bf16(proj, conv_state, conv_w)
    b = proj.shape[0]
    if proj.stride(-1) != 1:
        raise ValueError("proj must have unit column stride")
    if conv_state.shape != (b, 3, conv_dim) or not conv_state.is_contiguous():
        raise ValueError("conv_state must be contiguous [B, 3, conv_dim]")
    dev = N.require_device(proj, conv_state, conv_w, a_log, dt_bias)
    q = torch.empty(b, qk_dim, dtype=proj.dtype, device=dev)
    k = torch.empty_like(q)
    v = torch.empty(b, conv_dim - 2 * qk_dim, dtype=proj.dtype, device=dev)
    g = torch.empty(b, hv, dtype=torch.float32, device=dev)
    beta = torch.empty_like(g)
    N.call("yh_gdn_decode_prep", proj.data_ptr(), proj.stride(0), conv_state.data_ptr(), conv_w.data_ptr(),
           a_log.data_ptr(), dt_bias.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(),
           beta.data_ptr(), b, conv_dim, qk_dim, hv, b_offset, a_offset, 4, N.stream_of(proj))
    return q, k, v, g, beta


def gated_rmsnorm(o, z, w, eps):
    """Qwen3_5RMSNormGated (transformers wheel models/qwen3_5/modeling_qwen3_5.py:
    175-190) per head of 128: o [B, H, 128] contiguous, z a [B, H * 128] view
    (any row stride).  Returns [B, H * 128]."""
    _bf16(o, z, w)
    b, h, d = o.shape
    o = o.contiguous()
    if z.stride(-1) != 1:
        z = z.contiguous()
    N.require_device(o, z, w)
    out = torch.empty(b, h * d, dtype=o.dtype, device=o.device)
    N.call("yh_gated_rmsnorm", o.data_ptr(), z.data_ptr(), z.stride(0), w.data_ptr(), out.data_ptr(), b, h, d,
           float(eps), N.stream_of(o))
    return out


def silu_mul(gate_up):
    """silu(gate) * up of a packed [*, 2I] projection (runtime/model/
    inference_kernels.py:642-666); returns [*, I].  A 2-D input may be a
    column slice of a wider projection (any 16-byte aligned row stride)."""
    _bf16(gate_up)
    gu = gate_up
    if gu.ndim != 2 or gu.stride(-1) != 1 or gu.stride(0) % 8 or gu.data_ptr() % 16:
        gu = gu.contiguous().view(-1, gate_up.shape[-1])
    i2 = gu.shape[-1]
    n = gu.shape[0]
    N.require_device(gu)
    out = torch.empty(*gate_up.shape[:-1], i2 // 2, dtype=gu.dtype, device=gu.device)
    N.call("yh_silu_mul", gu.data_ptr(), gu.stride(0), out.data_ptr(), n, i2 // 2, N.stream_of(gu))
    return out


def head_norm_rope(x, w, cos, sin, rotary_dim, eps, *, out=None, out_tok_index=None, out_tok_stride=None,
                   out_head_stride=None):
    """Per-head RMSNorm (1 + w) then rotate-half RoPE on the first
    ``rotary_dim`` dims.  x [N, H, 128] (any token / head strides, unit last
    stride); cos / sin float [N, rotary_dim].  Writes a new [N, H, 128] tensor,
    or into ``out`` at row ``out_tok_index[n]`` with the given strides."""
    _bf16(x, w)
    n, h, d = x.shape
    if x.stride(-1) != 1:
        raise ValueError("x must have unit last stride")
    dev = N.require_device(x, w, cos, sin, out, out_tok_index)
    if out is None:
        out = torch.empty(n, h, d, dtype=x.dtype, device=dev)
        out_tok_stride, out_head_stride = h * d, d
    cs = None if cos is None else cos.float().contiguous()
    sn = None if sin is None else sin.float().contiguous()
    idx = None if out_tok_index is None else out_tok_index.to(torch.int64).contiguous()
    N.call("yh_head_norm_rope", x.data_ptr(), x.stride(0), x.stride(1), w.data_ptr(), N.ptr(cs), N.ptr(sn),
           out.data_ptr(), out_tok_stride, out_head_stride, N.ptr(idx), n, h, d, rotary_dim, float(eps),
           N.stream_of(x))
    return out


def ring_write(k, v, w, cos, sin, rows, positions, ring_k, ring_v, ring_pos, rotary_dim, eps):
    """Write one decode token per row into the SWA ring: the key heads k
    [N, H, 128] normed (1 + w) and rotated, the raw value heads v [N, H, 128]
    and positions [N] go to ring row ``rows[n]`` of ring_k / ring_v
    [N, H, W, 128] and ring_pos int32 [N, H, W]."""
    _bf16(k, v, w, ring_k, ring_v)
    n, h, d = k.shape
    if v.shape != k.shape or k.stride(-1) != 1 or v.stride(-1) != 1:
        raise ValueError("k / v must be [N, H, D] with unit last stride")
    if ring_k.ndim != 4 or ring_k.shape[1] != h or ring_k.shape[3] != d or ring_v.shape != ring_k.shape:
        raise ValueError("ring_k / ring_v must be [N, H, W, D]")
    if ring_pos.shape != ring_k.shape[:3] or ring_pos.dtype != torch.int32:
        raise ValueError("ring_pos must be int32 [N, H, W]")
    for t in (ring_k, ring_v, ring_pos):
        if not t.is_contiguous():
            raise ValueError("ring tensors must be contiguous")
    dev = N.require_device(k, v, w, cos, sin, rows, positions, ring_k)
    cs = None if cos is None else cos.float().contiguous()
    sn = None if sin is None else sin.float().contiguous()
    r = rows.to(torch.int64).contiguous()
    p = positions.to(torch.int64).contiguous()
    N.call("yh_ring_write", k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1),
           w.data_ptr(), N.ptr(cs), N.ptr(sn), r.data_ptr(), p.data_ptr(), ring_k.data_ptr(), ring_v.data_ptr(),
           ring_pos.data_ptr(), n, h, ring_k.shape[2], d, rotary_dim, float(eps), N.stream_of(k))


def memory_prologue(proj, heads, feat_offset, n_features, q_norm_w, cos, sin, read_scale, gate_w, gate_b, adm_up,
                    rotary_dim, eps, act_offset=None, act_width=0, act_out=None):
    """Query, read gate and admission scores of the anchor memory for one
    decode token per row from the fused projection proj [B, P] (query heads
    first, admission features at ``feat_offset``): returns q [B, H, 128] bf16,
    gate [B, H] float, scores [B, G] float (modeling_yanchor.py:167-176).
    With ``act_offset`` (the writer's gate columns, its up columns right
    after them, ``act_width`` each) the same launch also returns the writer's
    activation silu(gate) * up [B, act_width] bf16 as a fourth result, written
    into ``act_out`` when given (rows with unit last stride, any row stride)."""
    _bf16(proj, q_norm_w)
    b, ps = proj.shape
    if proj.stride(1) != 1:
        raise ValueError("proj must have unit last stride")
    g = adm_up.shape[0]
    dev = N.require_device(proj, q_norm_w, cos, sin, read_scale, gate_w, gate_b, adm_up)
    f32 = [t.to(torch.float32).contiguous() for t in (read_scale, gate_w, gate_b, adm_up)]
    cs = None if cos is None else cos.float().contiguous()
    sn = None if sin is None else sin.float().contiguous()
    q = torch.empty(b, heads, 128, dtype=proj.dtype, device=dev)
    gate = torch.empty(b, heads, dtype=torch.float32, device=dev)
    scores = torch.empty(b, g, dtype=torch.float32, device=dev)
    act = None
    if act_offset is not None:
        if act_out is not None:
            if act_out.shape != (b, act_width) or act_out.dtype != proj.dtype or act_out.stride(1) != 1:
                raise ValueError("act_out must be [B, act_width] in the projection dtype with unit last stride")
            N.require_device(act_out)
            act = act_out
        else:
            act = torch.empty(b, act_width, dtype=proj.dtype, device=dev)
    N.call("yh_memory_prologue", proj.data_ptr(), proj.stride(0), feat_offset, q_norm_w.data_ptr(), N.ptr(cs),
           N.ptr(sn), f32[0].data_ptr(), f32[1].data_ptr(), f32[2].data_ptr(), f32[3].data_ptr(), q.data_ptr(),
           gate.data_ptr(), scores.data_ptr(), b, heads, 128, g, n_features, rotary_dim, float(eps),
           0 if act is None else int(act_offset), int(act_width), N.ptr(act), 0 if act is None else act.stride(0),
           N.stream_of(proj))
    return (q, gate, scores) if act is None else (q, gate, scores, act)


def linear_silu(x, w):
    """The MLP activation F.silu(x . gate^T) * (x . up^T) in bf16 (torch
    rounding points kept) from a [gate; up] weight packed with pair_halves:
    x [M, K] bf16 (M <= 256) -> [M, N/2]."""
    if not isinstance(w, PackedWeight) or not w.pair_halves:
        raise ValueError("linear_silu takes a PackedWeight packed with pair_halves")
    _bf16(x)
    n, k = w.shape
    if x.ndim != 2 or x.shape[1] != k:
        raise ValueError("linear_silu expects x [M, K]")
    m = x.shape[0]
    if x.stride(1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    dev = N.require_device(x, w.data)
    out = torch.empty(m, n // 2, dtype=x.dtype, device=dev)
    N.call("yh_linear_packed", x.data_ptr(), x.stride(0), w.data.data_ptr(), out.data_ptr(), n // 2, m, n, k, None, 0,
           1, 1, None, 0, 0, None, N.stream_of(x))
    return out


_linear_ws: dict = {}


def _linear_workspace(device, nbytes):
    """Split-K workspace per (device, stream), grown on demand (every partial
    the reduce reads is written first, so it needs no clearing); projections
    on different streams never share one."""
    key = (device.index if device.index is not None else torch.cuda.current_device(),
           torch.cuda.current_stream(device).cuda_stream)
    ws = _linear_ws.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _linear_ws[key] = ws
    return ws


class PackedWeight:
    """A projection weight ``[N, K]`` bf16 repacked once into MFMA fragment
    order (yh_linear_pack), for the decode projection kernel: ``linear(x, pw)``
    takes it in place of the row-major weight.  N % 16 == 0, K % 128 == 0."""

    def __init__(self, w, pair_halves=False):
        """``pair_halves``: w is [gate; up] (two halves of N/2 rows) and the
        tiles are interleaved for ``linear_silu``."""
        _bf16(w)
        if w.ndim != 2 or w.shape[0] % (32 if pair_halves else 16) or w.shape[1] % 128:
            raise ValueError("packed weights need [N, K] with N % 16 (paired: 32) == 0 and K % 128 == 0")
        N.require_device(w)
        self.shape = tuple(w.shape)
        self.dtype = w.dtype
        self.pair_halves = bool(pair_halves)
        self.data = torch.empty(w.numel(), dtype=w.dtype, device=w.device)
        wc = w.contiguous()
        N.call("yh_linear_pack", wc.data_ptr(), self.data.data_ptr(), self.shape[0], self.shape[1],
               int(self.pair_halves), N.stream_of(wc))

    @staticmethod
    def fits(w, pair_halves=False):
        return (w.dtype == torch.bfloat16 and w.ndim == 2 and w.shape[0] % (32 if pair_halves else 16) == 0
                and w.shape[1] % 128 == 0)


class Partials:
    """A projection x . W^T (+ residual) still in S fp32 split-K planes
    ``part`` [S, M, N] in the stream's workspace: consume it with ``rmsnorm``
    (or ``reduce_partials``) before the next projection on the same stream.
    The residual is a bf16 [M, N] tensor, None, or a second projection's
    ``Partials`` (its own residual None), which the consumer sums and rounds
    to bf16 first: bf16(bf16(x . W^T) + bf16(x2 . W2^T))."""

    def __init__(self, part, residual):
        self.part, self.residual = part, residual
        self.shape = tuple(part.shape[1:])
        self.dtype = torch.bfloat16
        self.device = part.device


def reduce_partials(p):
    """``p`` summed as the projection's own reduce stores it: bf16 of the
    planes' sum in slice order, then bf16(that + residual) (yh_linear_reduce)."""
    r = p.residual
    if isinstance(r, Partials):
        r = reduce_partials(r)
    m, n = p.shape
    out = torch.empty(m, n, dtype=torch.bfloat16, device=p.device)
    if r is not None and (r.stride(-1) != 1 or r.stride(0) % 4 or r.data_ptr() % 8):   # 4-element reads
        r = r.contiguous()
    N.call("yh_linear_reduce", p.part.data_ptr(), out.data_ptr(), n, m, n, p.part.shape[0], N.ptr(r),
           0 if r is None else r.stride(0), N.stream_of(p.part))
    return out


def linear(x, w, split_k=None, residual=None, defer=False):
    """out = x . w^T for a decode batch (x [M, K] bf16 with M <= 256, w [N, K]
    bf16 or a PackedWeight): torch.nn.functional.linear without bias on the
    skinny-projection kernels; with ``residual`` ([M, N] bf16, unit last
    stride) out = bf16(x . w^T) + residual.  The split-K workspace is cached
    per (device, stream).  ``defer`` (packed weights): when K is split, return
    the fp32 partials as a ``Partials`` for ``rmsnorm`` to sum (one launch
    less)."""
    packed = isinstance(w, PackedWeight)
    if packed and w.pair_halves:
        raise ValueError("weights packed with pair_halves serve linear_silu")
    _bf16(x, w.data if packed else w, residual)
    if not packed and residual is not None:
        return linear(x, w, split_k) + residual
    n, kw = w.shape
    if x.ndim != 2 or (not packed and w.ndim != 2) or x.shape[1] != kw:
        raise ValueError("linear expects x [M, K] and w [N, K]")
    m, k = x.shape
    if x.stride(1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    wt = w.data if packed else w.contiguous()
    dev = N.require_device(x, wt)
    out = torch.empty(m, n, dtype=x.dtype, device=dev)
    if residual is not None:
        if residual.shape != (m, n) or residual.stride(1) != 1:
            raise ValueError("residual must be [M, N] with unit last stride")
        N.require_device(residual)
        if residual.stride(0) % 8 or residual.data_ptr() % 16:   # rows read 16 bytes at a time
            residual = residual.contiguous()
    if packed:
        s = int(split_k) if split_k is not None else N.lib().yh_linear_packed_split(m, n, k)
        nbytes = s * m * n * 4 if s > 1 else 0
        ws = _linear_workspace(dev, nbytes) if nbytes else None
        slices = ctypes.c_int64(1)
        N.call("yh_linear_packed", x.data_ptr(), x.stride(0), wt.data_ptr(), out.data_ptr(), n, m, n, k,
               N.ptr(residual), 0 if residual is None else residual.stride(0), 0, s, N.ptr(ws),
               0 if ws is None else ws.numel(), int(defer), ctypes.byref(slices), N.stream_of(x))
        if defer and slices.value > 1:
            part = ws[: slices.value * m * n * 4].view(torch.float32).view(slices.value, m, n)
            return Partials(part, residual)
        return out
    s = int(split_k) if split_k is not None else N.lib().yh_linear_split(m, n, k)
    nbytes = N.lib().yh_linear_workspace_bytes(m, n, k, s)
    ws = _linear_workspace(dev, nbytes) if nbytes else None
    N.call("yh_linear", x.data_ptr(), x.stride(0), wt.data_ptr(), out.data_ptr(), n, m, n, k, s, N.ptr(ws),
           0 if ws is None else ws.numel(), N.stream_of(x))
    return out


# ---------------------------------------------------------------------------
# Refill prefill of packed, ragged prompt pieces (cu_seqlens), each continuing
# its sequence's caches.

def _cu(cu_seqlens, device, total):
    """cu_seqlens (host or device) as int32 on the device, checked on the
    host (a prefill is not captured, so the copy is cheap): non-decreasing,
    from >= 0 to <= total, so no kernel reads past the packed tokens.  The
    small per-piece vectors (offsets, starts, ring rows) may come from the
    host; the activations and caches must be device tensors."""
    cu = cu_seqlens.to(device=device, dtype=torch.int32).contiguous()
    if cu.ndim != 1 or cu.numel() < 1:
        raise ValueError("cu_seqlens must be a 1-D offset vector")
    h = cu.cpu()
    if int(h[0]) != 0 or int(h[-1]) > total or bool((h[1:] < h[:-1]).any()):
        raise ValueError("cu_seqlens must be non-decreasing offsets from 0 within the packed tokens")
    return cu


def _pieces(starts, ring_rows, r, ring_batch, device):
    st = starts.to(device=device, dtype=torch.int64).contiguous()
    rr = ring_rows.to(device=device, dtype=torch.int64).contiguous()
    if st.shape != (r,) or rr.shape != (r,):
        raise ValueError("starts / ring_rows must hold one entry per piece")
    if r and (int(st.min()) < 0 or int(rr.max()) >= ring_batch):
        raise ValueError("starts must be >= 0 and ring rows inside the ring")
    return st, rr


def conv_prefill(proj, window, conv_w, cu_seqlens, channels):
    """The GDN layer's causal conv1d + SiLU over packed prompt pieces
    (the causal-conv1d prefill of the CUDA backend, modeling_yanchor.py:
    392-407): proj [N, >= channels] bf16 (the conv inputs are its first
    ``channels`` columns, any row stride), window [R, 3, channels] bf16, the
    inputs before each piece (zeros for a fresh sequence), updated IN PLACE
    to the last three inputs; conv_w [channels, 4].  Returns [N, channels]."""
    _bf16(proj, window, conv_w)
    n = proj.shape[0]
    dev = N.require_device(proj, window, conv_w)
    cu = _cu(cu_seqlens, dev, n)
    r = cu.numel() - 1
    if proj.ndim != 2 or proj.stride(1) != 1 or proj.shape[1] < channels:
        raise ValueError("proj must be [N, >= channels] with unit column stride")
    if window.shape != (r, 3, channels) or not window.is_contiguous():
        raise ValueError("window must be contiguous [R, 3, channels]")
    if conv_w.shape != (channels, 4) or not conv_w.is_contiguous():
        raise ValueError("conv_w must be contiguous [channels, 4]")
    if int(cu[-1]) != n:
        raise ValueError("cu_seqlens must cover every packed token")
    out = torch.empty(n, channels, dtype=proj.dtype, device=dev)
    N.call("yh_conv_prefill", proj.data_ptr(), proj.stride(0), window.data_ptr(), conv_w.data_ptr(), cu.data_ptr(),
           r, n, channels, out.data_ptr(), N.BF16, N.stream_of(proj))
    return out


def prefill_tiles(lengths, tokens_per_tile, device):
    """(piece, first token) int32 [n_tiles, 2] of the tiles of
    ``tokens_per_tile`` tokens that cover pieces of the given host lengths."""
    tiles = [(r, t) for r, n in enumerate(lengths) for t in range(0, int(n), tokens_per_tile)]
    return torch.tensor(tiles, dtype=torch.int32).reshape(-1, 2).to(device)


def _rows(x, name):
    """x [N, heads, 128] with unit head-dim stride, heads contiguous and
    16-byte aligned rows (a column view of a projection qualifies)."""
    if x.ndim != 3 or x.stride(2) != 1 or x.stride(1) != x.shape[2] or x.stride(0) % 8 or x.data_ptr() % 16:
        return x.contiguous()
    return x


def swa_prefill(q, k, v, cu_seqlens, starts, ring_k, ring_v, ring_rows, *, gate=None, lengths=None, tiles=None):
    """Sliding-window causal attention of packed prompt pieces (flash_swa /
    reference_swa, modeling_yanchor.py:412-449, with the output gate of
    871-875): query t of piece r at position starts[r] + t reads the
    ``window`` keys ending at its position, those before the piece from the
    ring row ``ring_rows[r]`` (slot = position % window).  q [N, H, 128]
    normed and rotated; k [N, G, 128] normed and rotated; v [N, G, 128];
    ring_k / ring_v [RB, G, window, 128]; starts / ring_rows int64 [R];
    gate None or [N, H, 128] (any token / head strides): the result is then
    read * sigmoid(gate).  Returns [N, H, 128]."""
    if q.dtype not in (torch.bfloat16, torch.float16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("swa_prefill takes bf16 / fp16 q, k, v")
    n, h, d = q.shape
    g = k.shape[1]
    if k.shape != (n, g, d) or v.shape != k.shape or h % g:
        raise ValueError("k / v must be [N, G, D] with G dividing the query heads")
    if ring_k.ndim != 4 or ring_k.shape[1] != g or ring_k.shape[3] != d or ring_v.shape != ring_k.shape:
        raise ValueError("ring_k / ring_v must be [RB, G, window, D]")
    if not ring_k.is_contiguous() or not ring_v.is_contiguous() or ring_k.dtype != q.dtype:
        raise ValueError("ring tensors must be contiguous in the query dtype")
    dev = N.require_device(q, k, v, ring_k, ring_v, gate)
    cu = _cu(cu_seqlens, dev, n)
    r = cu.numel() - 1
    st, rr = _pieces(starts, ring_rows, r, ring_k.shape[0], dev)
    if 64 % (h // g):
        raise ValueError("query heads per KV head must divide 64")
    lengths = (cu[1:] - cu[:-1]).tolist()
    if tiles is None:
        tiles = prefill_tiles(lengths, 64 // (h // g), dev)
    else:
        th = tiles.cpu()
        if tiles.dtype != torch.int32 or tiles.ndim != 2 or tiles.shape[1] != 2 or \
                any(not (0 <= int(p) < r and 0 <= int(t) < lengths[int(p)]) for p, t in th.tolist()):
            raise ValueError("tiles must be int32 (piece, first token) pairs inside the pieces")
        tiles = tiles.to(dev).contiguous()
    q, k, v = _rows(q, "q"), _rows(k, "k"), _rows(v, "v")
    gp, gts, ghs = None, 0, 0
    if gate is not None:
        if gate.shape != (n, h, d) or gate.stride(2) != 1 or gate.dtype != q.dtype:
            raise ValueError("gate must be [N, H, D] in the query dtype with unit last stride")
        gp, gts, ghs = gate.data_ptr(), gate.stride(0), gate.stride(1)
    out = torch.empty(n, h, d, dtype=q.dtype, device=dev)
    N.call("yh_swa_prefill", q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), v.data_ptr(), v.stride(0),
           ring_k.data_ptr(), ring_v.data_ptr(), rr.data_ptr(), st.data_ptr(), cu.data_ptr(), tiles.data_ptr(),
           tiles.shape[0], gp, gts, ghs, out.data_ptr(), r, ring_k.shape[0], h, g, d, ring_k.shape[2], N.code(q),
           N.stream_of(q))
    return out


def ring_fill(k, v, cu_seqlens, starts, ring_rows, ring_k, ring_v, ring_pos):
    """The last min(window, L) keys, values and positions of each packed
    piece into ring row ``ring_rows[r]`` at slot position % window (the ring
    a prefill leaves for the decode read).  k [N, G, 128] normed and rotated,
    v [N, G, 128]; ring_k / ring_v [RB, G, window, 128]; ring_pos int32
    [RB, G, window]."""
    if k.dtype not in (torch.bfloat16, torch.float16) or v.dtype != k.dtype or ring_k.dtype != k.dtype:
        raise ValueError("ring_fill takes bf16 / fp16 keys and values in the ring dtype")
    n, g, d = k.shape
    if v.shape != k.shape or ring_k.ndim != 4 or ring_k.shape[1] != g or ring_k.shape[3] != d or \
            ring_v.shape != ring_k.shape or ring_pos.shape != ring_k.shape[:3] or ring_pos.dtype != torch.int32:
        raise ValueError("ring_fill needs k / v [N, G, D], rings [RB, G, W, D] and int32 positions [RB, G, W]")
    for t in (ring_k, ring_v, ring_pos):
        if not t.is_contiguous():
            raise ValueError("ring tensors must be contiguous")
    dev = N.require_device(k, v, ring_k, ring_v, ring_pos)
    cu = _cu(cu_seqlens, dev, n)
    r = cu.numel() - 1
    st, rr = _pieces(starts, ring_rows, r, ring_k.shape[0], dev)
    k, v = _rows(k, "k"), _rows(v, "v")
    N.call("yh_ring_fill", k.data_ptr(), k.stride(0), v.data_ptr(), v.stride(0), rr.data_ptr(), st.data_ptr(),
           cu.data_ptr(), r, n, ring_k.data_ptr(), ring_v.data_ptr(), ring_pos.data_ptr(), g, d, ring_k.shape[2],
           N.code(k), N.stream_of(k))
