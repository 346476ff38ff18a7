"""Continuous-batching decode runtime over a random-init 4B-shaped YANchor model.

This is the workload that drives the hot path end to end: a Qwen3.5-style
hybrid stack where every 4th layer is sliding-window attention plus the
independent anchor memory and the others are Gated DeltaNet layers
(reference modeling_yanchor.py:877-964; layer pattern configuration_yanchor.py:
19).  Weights are random N(0, 0.02) bf16 (no checkpoint is available).

Per decode step (``Model.decode_step``): embedding, per layer RMSNorm and
projections on hipBLASLt (torch GEMMs), the GDN recurrent state update, the SWA
ring attention and the anchor read / commit on this package's HIP kernels,
final norm and lm_head, then sampling and slot bookkeeping on HIP kernels.  The
whole step is captured once into a HIP graph and replayed.

``Engine`` is the continuous-batching driver: Poisson arrivals, refill of
finished slots at poll points (a host sync, as in the reference), and the
reference's decode tokens/s definition -- useful decode token events (each
sequence's first token comes from prefill and is not counted) over
wall - initial prefill - refill prefill (runtime/inference.py:105-106,
180, 230-235; runtime/model/inference_kernels.py:1204, 1351-1765).
"""
from __future__ import annotations

import math
import time
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F


@dataclass
class ModelConfig:
    layers: int = 36
    hidden: int = 2560
    intermediate: int = 9728
    vocab: int = 151936
    gdn_heads_k: int = 32
    gdn_heads_v: int = 32
    gdn_dk: int = 128
    gdn_dv: int = 128
    conv_kernel: int = 4
    attn_heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    rotary_dim: int = 32           # partial rotary factor 0.25 of the head dim
    rope_theta: float = 1.0e7
    swa_window: int = 1024
    memory_capacity: int = 256
    memory_chunk: int = 64
    writer_intermediate: int = 2560
    admission_rank: int = 64
    memory_interval: int = 4       # layer i is SWA + memory when (i + 1) % interval == 0
    rms_eps: float = 1e-6
    init_std: float = 0.02

    def is_memory_layer(self, i: int) -> bool:
        return (i + 1) % self.memory_interval == 0

    @property
    def conv_dim(self) -> int:
        return 2 * self.gdn_heads_k * self.gdn_dk + self.gdn_heads_v * self.gdn_dv


# ---------------------------------------------------------------------------
# hot-path operations: the HIP kernels (default) -- a CPU restatement can be
# injected for a baseline run, nothing here imports one.

def _token_by_token_sequence(ops, q, key, value, scores, valid, chunk, state):
    """The decode read / commit sequence a prefill chunk stands for:
    q [B, L, H, D], key / value [B, L, G, D], scores [B, L, G]."""
    b, length = q.shape[:2]
    act = torch.ones(b, length, dtype=torch.bool, device=q.device) if valid is None else valid
    reads = []
    for t in range(length):
        reads.append(ops.memory_read(q[:, t:t + 1].contiguous(), state)[:, 0])
        ops.memory_commit(key[:, t:t + 1].contiguous(), value[:, t:t + 1].contiguous(), scores[:, t:t + 1],
                          act[:, t].contiguous(), chunk, state)
    if not reads:
        return q.new_zeros(q.shape)
    return torch.stack(reads, 1) * act[..., None, None].to(q.dtype)


class HipOps:
    """The package's HIP kernels behind the reference's call signatures."""

    def __init__(self):
        from . import gdn, independent_memory, inference_kernels, layers
        self.gdn = gdn
        self.mem = independent_memory
        self.ik = inference_kernels
        self.layers = layers

    # Fused decode-layer neighbours: HIP kernels for bf16 activations (the
    # served configuration).  A float32 model (used to pin the cache logic
    # without bf16 rounding) runs the torch formulations of the same layers.
    def rmsnorm(self, x, w, eps, residual=None, w2=None, w2_row=None):
        """x may be a projection's deferred split-K partials (``linear(...,
        defer=True)``): the reduce, the projection's residual, the residual
        add and the norms then run as one launch.  ``w2``: the row normed
        with a second weight is appended to the result (with ``w2_row``, as
        the first columns of rows that wide when one launch makes it)."""
        if x.dtype != torch.bfloat16:
            return TorchGlue.rmsnorm(x, w, eps, residual, w2)
        return self.layers.rmsnorm(x, w, eps, residual=residual, w2=w2, w2_row=w2_row)

    def gdn_prep(self, proj, conv_state, conv_w, a_log, dt_bias, **kw):
        if proj.dtype != torch.bfloat16:
            return TorchGlue.gdn_prep(proj, conv_state, conv_w, a_log, dt_bias, **kw)
        return self.layers.gdn_decode_prep(proj, conv_state, conv_w, a_log, dt_bias, **kw)

    def decode_inputs(self, tokens, positions, embed, w, inv_freq, eps, **kw):
        if embed.dtype != torch.bfloat16:
            return TorchGlue.decode_inputs(tokens, positions, embed, w, inv_freq, eps, **kw)
        return self.layers.decode_inputs(tokens, positions, embed, w, inv_freq, eps, **kw)

    def gdn_decode_fused(self, proj, conv_state, conv_w, a_log, dt_bias, state, norm_w, eps, **kw):
        """gdn_prep + gdn_decode + gated_rmsnorm of one decode token, one launch."""
        return self.layers.gdn_decode_fused(proj, conv_state, conv_w, a_log, dt_bias, state, norm_w, eps, **kw)

    def gated_rmsnorm(self, o, z, w, eps):
        if o.dtype != torch.bfloat16:
            return TorchGlue.gated_rmsnorm(o, z, w, eps)
        return self.layers.gated_rmsnorm(o, z, w, eps)

    def silu_mul(self, gate_up):
        if gate_up.dtype != torch.bfloat16:
            return TorchGlue.silu_mul(gate_up)
        return self.layers.silu_mul(gate_up)

    def head_norm_rope(self, x, w, cos, sin, rotary_dim, eps, **kw):
        if x.dtype != torch.bfloat16:
            return TorchGlue.head_norm_rope(x, w, cos, sin, rotary_dim, eps, **kw)
        return self.layers.head_norm_rope(x, w, cos, sin, rotary_dim, eps, **kw)

    # Decode projections on the packed-weight kernels (proj.hip), which beat
    # the library GEMM on MI355X at 128 rows (and at 256, the long-horizon
    # batch, for all but the fused k/v and the MLP gate/up, within 3 % there)
    # for every projection of the step
    # but the anchor memory's 2048-wide k/v (2048 x 5120 fused: 19.2 against
    # 15.3 us): the MLP, the GDN input and output, the attention q/k/v and
    # output, the memory's fused input and output projections, and the
    # lm_head.  Prefill (more rows) keeps the row-major weights.
    PACKED = ("mlp_gate_up", "mlp_down", "w_in", "w_out", "w_qkv", "w_o", "m_in", "m_o")

    # The anchor memory's key / value of a decode token in one projection:
    # kv = (u + write_down(act)) . W_kv^T = [u | act] . [W_kv | W_kv W_down]^T
    # (modeling_yanchor.py:147-166), the product W_kv W_down formed once in
    # float32 and rounded to the weights' dtype.  The reference rounds the
    # writer's output and the sum z to bf16 before the k / v projection; this
    # form rounds the product weight instead.  It takes two dependent
    # projections and a split-K reduce off the memory path, the longer of an
    # attention layer's two streams.  The row [u | act] is one buffer: the
    # norm writes u into its first columns and the prologue act into the rest.
    # bf16 weights only: a float32 model keeps the reference's order, so its
    # committed positions match the reference's exactly (a reassociation moves
    # near-tied admission scores at float32 rounding).
    fused_memory_kv = True

    def prepare(self, model):
        """Packed copies of the decode projection weights (``name + "@packed"``
        in each layer dict, ``model.lm_head_packed``); the row-major weights
        stay for prefill.  Attention layers also get ``m_kv@fused``, the fused
        memory k/v weight of the decode step.  These are copies: after the
        weights change, call prepare again."""
        for L in model.layers:
            if L.get("kind") == "attn" and "m_kv" in L and "writer_down" in L and L["m_kv"].dtype == torch.bfloat16:
                fused = (L["m_kv"].float() @ L["writer_down"].float()).to(L["m_kv"].dtype)
                L["m_kv@fused"] = torch.cat((L["m_kv"], fused), dim=1).contiguous()
            for name in self.PACKED:
                pair = name == "mlp_gate_up"   # [gate; up]: tiles interleaved for the fused silu * up
                if name in L and self.layers.PackedWeight.fits(L[name], pair):
                    L[name + "@packed"] = self.layers.PackedWeight(L[name], pair_halves=pair)
        if self.layers.PackedWeight.fits(model.lm_head):
            model.lm_head_packed = self.layers.PackedWeight(model.lm_head)

    def linear(self, x, w, packed=None, residual=None, defer=False):
        """out = x . w^T (+ residual, added to the bf16 product): the
        packed-weight kernel for a decode batch (bf16, <= 256 rows) when a
        packed copy exists, torch (hipBLASLt) otherwise.  ``defer``: the
        result is only ever fed to ``rmsnorm``, which may then do the split-K
        reduce itself.  Past 128 rows a K-split projection whose reduce would
        need a launch of its own stays on hipBLASLt (at 256 rows, 9280 x 2560:
        36.5 us against 28.5 + 14.5 for the split and its reduce)."""
        if packed is not None and x.dtype == torch.bfloat16 and x.ndim == 2 and x.shape[0] <= 256:
            m = x.shape[0]
            if m <= 128 or defer or self.layers.N.lib().yh_linear_packed_split(m, *packed.shape) == 1:
                return self.layers.linear(x, packed, residual=residual, defer=defer)
        out = F.linear(x, w)
        return out if residual is None else out + residual

    def add_projections(self, a, b):
        """a + b of two projections' results, as a projection's store adds its
        residual: bf16(bf16(a) + bf16(b)).  Deferred split-K partials stay
        partials for the norm that follows (``layers.Partials`` with the
        second as its residual); otherwise each is reduced as its own store
        would and the two are added."""
        P = self.layers.Partials
        if isinstance(a, P) and a.residual is None and (torch.is_tensor(b) or (
                isinstance(b, P) and b.residual is None and b.shape == a.shape)):
            return P(a.part, b)
        a = self.layers.reduce_partials(a) if isinstance(a, P) else a
        b = self.layers.reduce_partials(b) if isinstance(b, P) else b
        return a + b

    def mlp_act(self, x, w, packed=None):
        """silu(x . gate^T) * (x . up^T) of the [gate; up] MLP weight: one
        launch on the packed weights (decode batch), else GEMM + silu_mul."""
        if packed is not None and x.dtype == torch.bfloat16 and x.ndim == 2 and x.shape[0] <= 256:
            return self.layers.linear_silu(x, packed)
        return self.silu_mul(F.linear(x, w))

    def ring_write(self, k, v, w, cos, sin, rows, positions, ring_k, ring_v, ring_pos, rotary_dim, eps):
        if k.dtype != torch.bfloat16:
            return TorchGlue.ring_write(k, v, w, cos, sin, rows, positions, ring_k, ring_v, ring_pos, rotary_dim, eps)
        self.layers.ring_write(k, v, w, cos, sin, rows, positions, ring_k, ring_v, ring_pos, rotary_dim, eps)

    def memory_prologue(self, proj, heads, feat_offset, n_features, q_norm_w, cos, sin, read_scale, gate_w, gate_b,
                        adm_up, rotary_dim, eps):
        f = TorchGlue.memory_prologue if proj.dtype != torch.bfloat16 else self.layers.memory_prologue
        return f(proj, heads, feat_offset, n_features, q_norm_w, cos, sin, read_scale, gate_w, gate_b, adm_up,
                 rotary_dim, eps)

    def memory_prologue_act(self, proj, heads, feat_offset, n_features, q_norm_w, cos, sin, read_scale, gate_w,
                            gate_b, adm_up, rotary_dim, eps, act_offset, act_width, act_out=None):
        """memory_prologue plus the writer's silu(gate) * up in the same
        launch (bf16; otherwise the two separate ops), into ``act_out`` when
        given."""
        if proj.dtype != torch.bfloat16:
            out = TorchGlue.memory_prologue(proj, heads, feat_offset, n_features, q_norm_w, cos, sin, read_scale,
                                            gate_w, gate_b, adm_up, rotary_dim, eps)
            act = self.silu_mul(proj[:, act_offset: act_offset + 2 * act_width])
            if act_out is not None:
                act_out.copy_(act)
                act = act_out
            return out + (act,)
        return self.layers.memory_prologue(proj, heads, feat_offset, n_features, q_norm_w, cos, sin, read_scale,
                                           gate_w, gate_b, adm_up, rotary_dim, eps, act_offset=act_offset,
                                           act_width=act_width, act_out=act_out)

    def gdn_decode(self, q, k, v, g, beta, state):
        o, _ = self.gdn.recurrent_gated_delta_rule(q, k, v, g=g, beta=beta, initial_state=state,
                                                   output_final_state=True, use_qk_l2norm_in_kernel=True)
        return o

    def gdn_prefill(self, q, k, v, g, beta, cu_seqlens, lengths, initial_state=None):
        """Packed pieces [1, N, ...] of cu_seqlens from ``initial_state``
        ([R, HV, K, V], None = zeros): one chunk-kernel launch (bf16) or the
        token-recurrent kernel (other dtypes); returns (o, final states)."""
        return self.gdn.chunk_gated_delta_rule(q, k, v, g=g, beta=beta, initial_state=initial_state,
                                               output_final_state=True, use_qk_l2norm_in_kernel=True,
                                               cu_seqlens=cu_seqlens, lengths=lengths)

    def conv_prefill(self, proj, window, conv_w, cu_seqlens, channels, lengths):
        if proj.dtype != torch.bfloat16:
            return TorchGlue.conv_prefill(proj, window, conv_w, cu_seqlens, channels, lengths)
        return self.layers.conv_prefill(proj, window, conv_w, cu_seqlens, channels)

    def swa_prefill(self, q, k, v, cu_seqlens, starts, ring_k, ring_v, ring_rows, gate=None, lengths=None):
        if q.dtype not in (torch.bfloat16, torch.float16):
            return TorchGlue.swa_prefill(q, k, v, cu_seqlens, starts, ring_k, ring_v, ring_rows, gate, lengths)
        return self.layers.swa_prefill(q, k, v, cu_seqlens, starts, ring_k, ring_v, ring_rows, gate=gate,
                                       lengths=lengths)

    def ring_fill(self, k, v, cu_seqlens, starts, ring_rows, ring_k, ring_v, ring_pos, lengths=None):
        if k.dtype not in (torch.bfloat16, torch.float16):
            return TorchGlue.ring_fill(k, v, cu_seqlens, starts, ring_rows, ring_k, ring_v, ring_pos, lengths)
        self.layers.ring_fill(k, v, cu_seqlens, starts, ring_rows, ring_k, ring_v, ring_pos)

    def window_attend(self, q, keys, values, positions, gate=None):
        return self.mem.ring_decode_attention(q, keys, values, positions, gate=gate)

    def memory_read(self, q, state, valid=None, head_gate=None):
        return self.mem.committed_gqa_gated(q, state, None, valid, head_gate)

    def memory_commit(self, key, value, scores, active, chunk, state):
        self.mem.commit_decode(key, value, scores, active, chunk, state)

    def memory_sequence(self, q, key, value, scores, valid, chunk, state):
        """Prefill read + write continuing ``state`` (_sequence).  The block
        kernels take 16-bit K/V; fp32 memories run the decode kernels token by
        token, which read and leave the same."""
        if q.dtype in (torch.bfloat16, torch.float16):
            return self.mem.sequence(q, key, value, scores, valid, chunk, state)
        return _token_by_token_sequence(self, q, key, value, scores, valid, chunk, state)

    def sample(self, logits, attempt_ids, steps, seen, *, seed, temperature, top_k, top_p, penalty,
               backend="triton_top20"):
        """One token per row with the presence penalty of ``seen`` fused in:
        the fused top-k kernel's semantics ("triton_top20") or the torch
        sampler's ("torch", any top_k)."""
        mode = self.ik.SAMPLE_FUSED if backend == "triton_top20" else self.ik.SAMPLE_TORCH
        return self.ik.topk_sample(logits, attempt_ids, steps, seed=seed, temperature=temperature, top_k=top_k,
                                   top_p=top_p, mode=mode, seen=seen, presence_penalty=penalty)

    def bookkeeping(self, *args, **kw):
        self.ik._update_fixed_decode_state_(*args, **kw)


# ---------------------------------------------------------------------------

def rms_norm(x, w, eps, plus_one=True):
    """Qwen3.5 RMSNorm: x / rms(x) * (1 + w), computed in fp32."""
    xf = x.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    y = y * ((1.0 + w.float()) if plus_one else w.float())
    return y.to(x.dtype)


def gated_rms_norm(x, gate, w, eps):
    """Qwen3_5RMSNormGated (transformers wheel models/qwen3_5/modeling_qwen3_5.py:
    175-184): normalise in fp32, round, scale by w in the weight dtype, times
    silu(gate) in fp32."""
    xf = x.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    y = (w * y.to(x.dtype)).float() * F.silu(gate.float())
    return y.to(x.dtype)


def rope_inv_freq(cfg: ModelConfig, device):
    """theta^(-j / half) for j < rotary_dim / 2, float32."""
    half = cfg.rotary_dim // 2
    return 1.0 / (cfg.rope_theta ** (torch.arange(0, half, device=device, dtype=torch.float32) / half))


def rope_tables(positions, cfg: ModelConfig):
    """cos / sin [*, rotary_dim] for integer positions (rotate_half layout)."""
    ang = positions.float()[..., None] * rope_inv_freq(cfg, positions.device)
    ang = torch.cat((ang, ang), -1)
    return ang.cos(), ang.sin()


def apply_rope(x, cos, sin, rd):
    """Rotate the first rd dims of x [..., D] (cos/sin broadcast over heads)."""
    xr = x[..., :rd].float()
    x1, x2 = xr[..., : rd // 2], xr[..., rd // 2:]
    rot = torch.cat((-x2, x1), -1)
    out = xr * cos + rot * sin
    return torch.cat((out.to(x.dtype), x[..., rd:]), -1)


class TorchGlue:
    """Torch formulations of the fused decode-layer kernels, argument for
    argument (the definitions the kernels are tested against)."""

    @staticmethod
    def rmsnorm(x, w, eps, residual=None, w2=None):
        s = x if residual is None else x + residual
        res = (rms_norm(s, w, eps),) if residual is None else (rms_norm(s, w, eps), s)
        res = res if w2 is None else res + (rms_norm(s, w2, eps),)
        return res[0] if len(res) == 1 else res

    @staticmethod
    def decode_inputs(tokens, positions, embed, w, inv_freq, eps, *, ring_stride, window, finished=None,
                      slot_rows=None):
        h = embed[tokens]
        ang = positions.float()[:, None] * inv_freq
        ang = torch.cat((ang, ang), -1)
        rows = torch.arange(tokens.shape[0], device=tokens.device) * ring_stride + positions % window
        valid = None if finished is None else (~finished) & (slot_rows >= 0)
        return h, rms_norm(h, w, eps), ang.cos(), ang.sin(), rows, valid

    @staticmethod
    def gdn_prep(proj, conv_state, conv_w, a_log, dt_bias, *, conv_dim, qk_dim, hv, b_offset, a_offset):
        window = torch.cat((conv_state, proj[:, None, :conv_dim]), 1)          # [B, K, C], oldest first
        conv_state.copy_(window[:, 1:])
        mixed = F.silu((window.float() * conv_w.float().t()[None]).sum(1)).to(proj.dtype)
        b = proj[:, b_offset: b_offset + hv]
        beta = torch.sigmoid(b.float()).to(b.dtype).float()         # beta in the logits' dtype
        g = -torch.exp(a_log) * F.softplus(proj[:, a_offset: a_offset + hv].float() + dt_bias)
        return mixed[:, :qk_dim], mixed[:, qk_dim: 2 * qk_dim], mixed[:, 2 * qk_dim:], g, beta

    @staticmethod
    def gated_rmsnorm(o, z, w, eps):
        b, h, d = o.shape
        return gated_rms_norm(o, z.reshape(b, h, d), w, eps).reshape(b, h * d)

    @staticmethod
    def silu_mul(gate_up):
        gate, up = gate_up.chunk(2, -1)
        return F.silu(gate) * up

    @staticmethod
    def head_norm_rope(x, w, cos, sin, rotary_dim, eps, *, out=None, out_tok_index=None, out_tok_stride=None,
                       out_head_stride=None):
        y = rms_norm(x, w, eps)
        if rotary_dim:
            y = apply_rope(y, cos[:, None], sin[:, None], rotary_dim)
        if out is None:
            return y
        n, h, d = y.shape
        rows = (out.numel() - (h - 1) * out_head_stride - d) // out_tok_stride + 1
        dst = out.as_strided((rows, h, d), (out_tok_stride, out_head_stride, 1))
        dst[out_tok_index] = y
        return out


def _torch_ring_write(k, v, w, cos, sin, rows, positions, ring_k, ring_v, ring_pos, rotary_dim, eps):
    n, h, d = k.shape
    window = ring_k.shape[2]
    TorchGlue.head_norm_rope(k, w, cos, sin, rotary_dim, eps, out=ring_k, out_tok_index=rows, out_tok_stride=d,
                             out_head_stride=window * d)
    slot = positions % window
    tok = torch.arange(n, device=k.device)
    ring_v[tok, :, slot] = v
    ring_pos[tok, :, slot] = positions.to(torch.int32)[:, None]


def _torch_memory_prologue(proj, heads, feat_offset, n_features, q_norm_w, cos, sin, read_scale, gate_w, gate_b,
                           adm_up, rotary_dim, eps):
    b = proj.shape[0]
    d = 128
    mq = proj[:, : heads * d].view(b, heads, d)
    qn = TorchGlue.head_norm_rope(mq, q_norm_w, None, None, 0, eps)
    gate = torch.tanh(read_scale) * 2 * torch.sigmoid((qn.float() * gate_w).sum(-1) / math.sqrt(d) + gate_b)
    q = TorchGlue.head_norm_rope(mq, q_norm_w, cos, sin, rotary_dim, eps)
    scores = F.linear(F.silu(proj[:, feat_offset: feat_offset + n_features]).float(), adm_up)
    return q, gate, scores


def _torch_conv_prefill(proj, window, conv_w, cu_seqlens, channels, lengths):
    """Causal conv1d + SiLU over packed pieces, each continuing its row's
    window [R, 3, C] (updated in place): fp32 taps, one rounding."""
    x = proj[:, :channels]
    outs, off = [], 0
    for r, n in enumerate(lengths):
        ext = torch.cat((window[r], x[off: off + n].to(window.dtype)), 0)             # [3 + n, C]
        if n:
            y = sum(ext[j: j + n].float() * conv_w[:, j].float() for j in range(conv_w.shape[1]))
            outs.append(F.silu(y).to(proj.dtype))
        window[r].copy_(ext[n:])
        off += n
    return torch.cat(outs) if outs else proj.new_zeros(0, channels)


def _ring_context(ring, row, start, window):
    """The min(start, window - 1) ring entries before position ``start`` of
    ring row ``row`` [G, W, ...], oldest first, as [n, G, ...]."""
    n = min(start, window - 1) if row >= 0 else 0
    slots = torch.arange(start - n, start, device=ring.device) % window
    return ring[row][:, slots].transpose(0, 1) if n else ring.new_zeros((0,) + (ring.shape[1],) + ring.shape[3:])


def _torch_swa_prefill(q, k, v, cu_seqlens, starts, ring_k, ring_v, ring_rows, gate=None, lengths=None):
    """Sliding-window causal attention of packed pieces with the ring as
    left context (reference_swa, modeling_yanchor.py:412-427), fp32, query
    blocks of 1024; then * sigmoid(gate)."""
    n, h, d = q.shape
    g, window = k.shape[1], ring_k.shape[2]
    rep = h // g
    cu = cu_seqlens.tolist()
    lengths = lengths if lengths is not None else [cu[i + 1] - cu[i] for i in range(len(cu) - 1)]
    st, rr = starts.tolist(), ring_rows.tolist()
    out = torch.empty_like(q)
    off = 0
    for r, length in enumerate(lengths):
        if length:
            kc = torch.cat((_ring_context(ring_k, rr[r], st[r], window), k[off: off + length]), 0)
            vc = torch.cat((_ring_context(ring_v, rr[r], st[r], window), v[off: off + length]), 0)
            nctx = kc.shape[0] - length
            for b0 in range(0, length, 1024):
                b1 = min(length, b0 + 1024)
                lo, hi = max(0, nctx + b0 - window + 1), nctx + b1
                qp = torch.arange(nctx + b0, nctx + b1, device=q.device)
                kp = torch.arange(lo, hi, device=q.device)
                mask = (kp[None] <= qp[:, None]) & (kp[None] > qp[:, None] - window)
                kb = kc[lo:hi].float().repeat_interleave(rep, 1)
                vb = vc[lo:hi].float().repeat_interleave(rep, 1)
                logits = torch.einsum("lhd,shd->hls", q[off + b0: off + b1].float(), kb) / math.sqrt(d)
                p = logits.masked_fill(~mask[None], -math.inf).softmax(-1)
                out[off + b0: off + b1] = torch.einsum("hls,shd->lhd", p, vb).to(q.dtype)
        off += length
    return out if gate is None else out * torch.sigmoid(gate)


def _torch_ring_fill(k, v, cu_seqlens, starts, ring_rows, ring_k, ring_v, ring_pos, lengths=None):
    """The last min(window, L) keys / values / positions of each packed piece
    into its ring row at slot position % window."""
    window = ring_k.shape[2]
    cu = cu_seqlens.tolist()
    lengths = lengths if lengths is not None else [cu[i + 1] - cu[i] for i in range(len(cu) - 1)]
    st, rr = starts.tolist(), ring_rows.tolist()
    off = 0
    for r, length in enumerate(lengths):
        if length and rr[r] >= 0:
            t = torch.arange(max(0, length - window), length, device=k.device)
            pos = st[r] + t
            slots = pos % window
            ring_k[rr[r]][:, slots] = k[off + t].transpose(0, 1).to(ring_k.dtype)
            ring_v[rr[r]][:, slots] = v[off + t].transpose(0, 1).to(ring_v.dtype)
            ring_pos[rr[r]][:, slots] = pos.to(torch.int32)[None]
        off += length


TorchGlue.ring_write = staticmethod(_torch_ring_write)
TorchGlue.memory_prologue = staticmethod(_torch_memory_prologue)
TorchGlue.conv_prefill = staticmethod(_torch_conv_prefill)
TorchGlue.swa_prefill = staticmethod(_torch_swa_prefill)
TorchGlue.ring_fill = staticmethod(_torch_ring_fill)


def gate_read(read, valid=None, head_gate=None, gate=None):
    """The torch formulation of the decode layer's gating of a read
    [B, 1, H, D]: (read * valid) * head_gate, or read * sigmoid(gate)."""
    if valid is not None:
        read = read * valid[:, None, None, None].to(read.dtype)
    if head_gate is not None:
        read = read * head_gate[:, None, :, None].to(read.dtype)
    if gate is not None:
        read = read * torch.sigmoid(gate)[:, None]
    return read


class Model:
    """Random-init 4B-shaped hybrid recurrent model with its decode caches."""

    def __init__(self, cfg: ModelConfig, batch: int, device, *, seed=0, ops=None, dtype=torch.bfloat16,
                 init="normal", overlap=True, state_dtype=torch.float32):
        """``init="normal"`` draws every weight from N(0, init_std);
        ``init="tiled"`` repeats one 16M-value N(0, init_std) block (fast on a
        host, for timing runs where the values do not matter).
        ``state_dtype``: the GDN recurrent state's storage, float32 or float16
        (the reference's throughput profile: convert_fixed_memory_recurrent_
        state_storage_, modeling_yanchor.py:733-750; bf16 models only)."""
        if state_dtype not in (torch.float32, torch.float16):
            raise ValueError("the GDN state is stored as float32 or float16")
        if state_dtype != torch.float32 and (dtype != torch.bfloat16 or cfg.gdn_heads_k != cfg.gdn_heads_v
                                            or not cfg.gdn_dk == cfg.gdn_dv == 128):
            raise ValueError("a float16 GDN state needs a bfloat16 model whose GDN layers take the fused decode "
                             "core (as many key as value heads, 128-dim heads)")
        self.cfg, self.B, self.device, self.dtype = cfg, int(batch), torch.device(device), dtype
        self.state_dtype = state_dtype
        self.ops = ops if ops is not None else HipOps()
        self.overlap = overlap
        self._side = None
        gen = torch.Generator(device=self.device).manual_seed(seed)
        std = cfg.init_std
        block = None
        if init == "tiled":
            block = (torch.randn(1 << 24, device=self.device, generator=gen) * std).to(dtype)
        elif init != "normal":
            raise ValueError(f"unknown init {init!r}")

        def w(*shape):
            if block is not None:
                n, bn = math.prod(shape), block.numel()
                out = torch.empty(n, device=self.device, dtype=dtype)
                full = n // bn * bn
                out[:full].view(-1, bn).copy_(block.expand(n // bn, bn))
                out[full:].copy_(block[: n - full])
                return out.view(*shape)
            return (torch.randn(*shape, device=self.device, generator=gen, dtype=torch.float32) * std).to(dtype)

        def zeros(*shape):
            return torch.zeros(*shape, device=self.device, dtype=dtype)

        c = cfg
        self.inv_freq = rope_inv_freq(c, self.device)
        self.embed = w(c.vocab, c.hidden)
        self.lm_head = w(c.vocab, c.hidden)
        self.final_norm = zeros(c.hidden)
        self.layers = []
        for i in range(c.layers):
            L = {"in_norm": zeros(c.hidden), "post_norm": zeros(c.hidden),
                 "mlp_gate_up": w(2 * c.intermediate, c.hidden), "mlp_down": w(c.hidden, c.intermediate)}
            if c.is_memory_layer(i):
                qkv_out = 2 * c.attn_heads * c.head_dim + 2 * c.kv_heads * c.head_dim
                L.update(kind="attn", w_qkv=w(qkv_out, c.hidden), q_norm=zeros(c.head_dim),
                         k_norm=zeros(c.head_dim), w_o=w(c.hidden, c.attn_heads * c.head_dim),
                         m_in_norm=zeros(c.hidden),
                         m_q_norm=zeros(c.head_dim), m_k_norm=zeros(c.head_dim),
                         read_scale=w(c.attn_heads).float(), read_gate_w=w(c.attn_heads, c.head_dim).float(),
                         read_gate_b=w(c.attn_heads).float(),
                         writer_down=w(c.hidden, c.writer_intermediate),
                         m_kv=w(2 * c.kv_heads * c.head_dim, c.hidden),
                         adm_up=w(c.kv_heads, c.admission_rank).float(),
                         m_o=w(c.hidden, c.attn_heads * c.head_dim))
                # the three projections of u (query, admission features, writer
                # gate|up) share one weight so the decode step runs one GEMM
                qd, ad = c.attn_heads * c.head_dim, c.admission_rank
                m_in = w(qd + ad + 2 * c.writer_intermediate, c.hidden)
                L.update(m_in=m_in, m_q=m_in[:qd], adm_down=m_in[qd: qd + ad], writer_gate_up=m_in[qd + ad:])
            else:
                in_out = c.conv_dim + c.gdn_heads_v * c.gdn_dv + 2 * c.gdn_heads_v
                a_log = torch.log(torch.empty(c.gdn_heads_v, device=self.device).uniform_(1.0, 16.0,
                                                                                          generator=gen))
                L.update(kind="gdn", w_in=w(in_out, c.hidden), conv_w=w(c.conv_dim, c.conv_kernel),
                         a_log=a_log, dt_bias=torch.ones(c.gdn_heads_v, device=self.device),
                         gnorm=torch.ones(c.gdn_dv, device=self.device, dtype=dtype),
                         w_out=w(c.hidden, c.gdn_heads_v * c.gdn_dv))
            self.layers.append(L)
        self.lm_head_packed = None
        prepare = getattr(self.ops, "prepare", None)
        if prepare is not None:
            prepare(self)
        self._alloc_caches()

    # ---------------- caches ----------------
    def _alloc_caches(self):
        c, B, dev = self.cfg, self.B, self.device
        self.gdn_state, self.conv_state, self.ring_k, self.ring_v, self.ring_pos, self.memory = {}, {}, {}, {}, {}, {}
        from .independent_memory import IndependentMemoryState
        for i, L in enumerate(self.layers):
            if L["kind"] == "gdn":
                self.gdn_state[i] = torch.zeros(B, c.gdn_heads_v, c.gdn_dk, c.gdn_dv, device=dev,
                                                dtype=self.state_dtype)
                # time-major [B, K-1, C]: the decode prologue reads one coalesced row per tap
                self.conv_state[i] = torch.zeros(B, c.conv_kernel - 1, c.conv_dim, device=dev, dtype=self.dtype)
            else:
                self.ring_k[i] = torch.zeros(B, c.kv_heads, c.swa_window, c.head_dim, device=dev, dtype=self.dtype)
                self.ring_v[i] = torch.zeros_like(self.ring_k[i])
                self.ring_pos[i] = torch.full((B, c.kv_heads, c.swa_window), -1, device=dev, dtype=torch.int32)
                self.memory[i] = IndependentMemoryState.empty(B, c.kv_heads, c.memory_capacity, c.memory_chunk,
                                                              c.head_dim, dev, self.dtype)

    def cache_tensors(self):
        """Every per-slot cache tensor (dim 0 = slot), for refill and compaction."""
        from dataclasses import fields as dfields
        out = []
        for i in self.gdn_state:
            out += [self.gdn_state[i], self.conv_state[i]]
        for i in self.ring_k:
            out += [self.ring_k[i], self.ring_v[i], self.ring_pos[i]]
            st = self.memory[i]
            out += [getattr(st, f.name) for f in dfields(st)]
        return out

    # ---------------- layers ----------------
    def _mlp(self, L, x, defer=False):
        ops = self.ops
        return ops.linear(ops.mlp_act(x, L["mlp_gate_up"], L.get("mlp_gate_up@packed")), L["mlp_down"],
                          L.get("mlp_down@packed"), defer=defer)

    def _gdn_split(self, L, proj):
        c = self.cfg
        qkv = proj[..., : c.conv_dim]
        z = proj[..., c.conv_dim: c.conv_dim + c.gdn_heads_v * c.gdn_dv]
        b = proj[..., c.conv_dim + c.gdn_heads_v * c.gdn_dv: c.conv_dim + c.gdn_heads_v * c.gdn_dv + c.gdn_heads_v]
        a = proj[..., -c.gdn_heads_v:]
        beta = torch.sigmoid(b.float()).to(b.dtype).float()          # beta in the logits' dtype (wheel:500)
        g = -torch.exp(L["a_log"]) * F.softplus(a.float() + L["dt_bias"])
        return qkv, z, beta, g

    def _gdn_decode(self, i, L, xn):
        """GDN mixer for one token per slot; xn is the normalised layer input."""
        c, B, ops = self.cfg, xn.shape[0], self.ops
        hv, dv, vd = c.gdn_heads_v, c.gdn_dv, c.gdn_heads_v * c.gdn_dv
        proj = self.ops.linear(xn, L["w_in"], L.get("w_in@packed"))                                     # [B, qkv | z | b | a]
        if proj.dtype == torch.bfloat16 and hasattr(ops, "gdn_decode_fused") and c.gdn_heads_k == hv and \
                c.gdn_dk == dv == 128:
            y = ops.gdn_decode_fused(proj, self.conv_state[i], L["conv_w"], L["a_log"], L["dt_bias"],
                                     self.gdn_state[i], L["gnorm"], c.rms_eps, heads=hv, head_dim=dv,
                                     z_offset=c.conv_dim, b_offset=c.conv_dim + vd, a_offset=c.conv_dim + vd + hv)
            return self.ops.linear(y, L["w_out"], L.get("w_out@packed"), defer=True)
        q, k, v, g, beta = ops.gdn_prep(proj, self.conv_state[i], L["conv_w"], L["a_log"], L["dt_bias"],
                                        conv_dim=c.conv_dim, qk_dim=c.gdn_heads_k * c.gdn_dk, hv=hv,
                                        b_offset=c.conv_dim + vd, a_offset=c.conv_dim + vd + hv)
        o = ops.gdn_decode(q.view(B, 1, c.gdn_heads_k, c.gdn_dk), k.view(B, 1, c.gdn_heads_k, c.gdn_dk),
                           v.view(B, 1, hv, dv), g[:, None], beta[:, None], self.gdn_state[i])
        y = ops.gated_rmsnorm(o.view(B, hv, dv), proj[:, c.conv_dim: c.conv_dim + vd], L["gnorm"], c.rms_eps)
        return self.ops.linear(y, L["w_out"], L.get("w_out@packed"), defer=True)

    def _memory_qkvs(self, L, hidden, cos, sin):
        """_query_scores + _write_kv of IndependentGQAMemory (modeling_yanchor.py:147-176)."""
        c = self.cfg
        u = rms_norm(hidden, L["m_in_norm"], c.rms_eps)
        q = rms_norm(F.linear(u, L["m_q"]).unflatten(-1, (c.attn_heads, c.head_dim)), L["m_q_norm"], c.rms_eps)
        gate = torch.tanh(L["read_scale"]) * 2 * torch.sigmoid(
            (q.float() * L["read_gate_w"]).sum(-1) / math.sqrt(c.head_dim) + L["read_gate_b"])
        q = apply_rope(q, cos, sin, c.rotary_dim)
        feats = F.silu(F.linear(u, L["adm_down"]))
        scores = F.linear(feats.float(), L["adm_up"])
        gu = F.linear(u, L["writer_gate_up"])
        wg, wu = gu.chunk(2, -1)
        zz = u + F.linear(F.silu(wg) * wu, L["writer_down"])
        kv = F.linear(zz, L["m_kv"])
        key = kv[..., : c.kv_heads * c.head_dim].unflatten(-1, (c.kv_heads, c.head_dim))
        val = kv[..., c.kv_heads * c.head_dim:].unflatten(-1, (c.kv_heads, c.head_dim))
        key = apply_rope(rms_norm(key, L["m_k_norm"], c.rms_eps), cos, sin, c.rotary_dim)
        return q, gate, key, val.contiguous(), scores

    def _memory_decode(self, L, hidden, cos, sin, u=None):
        """``_memory_qkvs`` for one token per slot on the fused kernels (u:
        the layer input already normed with m_in_norm, if the previous norm
        made it)."""
        c, B, ops = self.cfg, hidden.shape[0], self.ops
        H, KVH, D = c.attn_heads, c.kv_heads, c.head_dim
        if u is None:
            u = ops.rmsnorm(hidden, L["m_in_norm"], c.rms_eps)
        proj = ops.linear(u, L["m_in"], L.get("m_in@packed"))                                    # [q | admission features | gate | up]
        qd, ad = H * D, c.admission_rank
        args = (proj, H, qd, ad, L["m_q_norm"], cos, sin, L["read_scale"], L["read_gate_w"], L["read_gate_b"],
                L["adm_up"], c.rotary_dim, c.rms_eps)
        if getattr(ops, "fused_memory_kv", False) and "m_kv@fused" in L:
            ua = self._memory_row(u)
            q, gate, scores, _ = ops.memory_prologue_act(*args, qd + ad, c.writer_intermediate,
                                                         act_out=ua[:, c.hidden:])
            kv = ops.linear(ua, L["m_kv@fused"])
        else:
            if hasattr(ops, "memory_prologue_act"):   # the writer's activation in the same launch
                q, gate, scores, act = ops.memory_prologue_act(*args, qd + ad, c.writer_intermediate)
            else:
                q, gate, scores = ops.memory_prologue(*args)
                act = ops.silu_mul(proj[:, qd + ad:])
            zz = ops.linear(act, L["writer_down"], L.get("writer_down@packed"), residual=u)
            kv = ops.linear(zz, L["m_kv"], L.get("m_kv@packed"))
        key = ops.head_norm_rope(kv[:, : KVH * D].view(B, KVH, D), L["m_k_norm"], cos, sin, c.rotary_dim,
                                 c.rms_eps)
        return q, gate, key, kv[:, KVH * D:].reshape(B, KVH, D), scores

    def _memory_row(self, u):
        """The [u | act] rows of the fused memory k/v projection: in place
        when u is the first columns of a [B, hidden + writer_intermediate]
        buffer of its own (the norm's ``w2_row`` output, whose other columns
        hold nothing), else a copy into a new buffer."""
        c = self.cfg
        width = c.hidden + c.writer_intermediate
        b = u.shape[0]
        base = u._base
        if (base is not None and base.shape == (b, width) and base.is_contiguous() and base.dtype == u.dtype
                and u.stride() == (width, 1) and u.data_ptr() == base.data_ptr()):
            return base
        ua = torch.empty(b, width, dtype=u.dtype, device=u.device)
        ua[:, : c.hidden].copy_(u)
        return ua

    def _attn_decode(self, i, L, xn, hidden, positions, cos, sin, valid, ring_rows, u=None):
        """SWA + anchor-memory mixer for one token per slot.  xn is the
        normalised layer input, hidden the residual stream entering the layer;
        ring_rows[b] = b * kv_heads * window + positions[b] % window.  On a GPU
        the memory path (its own norm, projections, read, commit and output
        projection) runs on a second stream beside the SWA path.  The two
        output projections meet in the norm after the layer, which sums their
        split-K partials, so neither waits for the other stream."""
        c, B, ops = self.cfg, xn.shape[0], self.ops
        H, KVH, D = c.attn_heads, c.kv_heads, c.head_dim
        side = self._side_stream(xn)
        if side is not None:
            main = torch.cuda.current_stream(xn.device)
            side.wait_stream(main)
            with torch.cuda.stream(side):
                mo = self._memory_out(i, L, hidden, cos, sin, valid, u)
        proj = ops.linear(xn, L["w_qkv"], L.get("w_qkv@packed"))                                    # [B, (q|gate) per head | k | v]
        hq = 2 * H * D
        qg = proj[:, :hq].view(B, H, 2 * D)
        q = ops.head_norm_rope(qg[..., :D], L["q_norm"], cos, sin, c.rotary_dim, c.rms_eps)
        ops.ring_write(proj[:, hq: hq + KVH * D].view(B, KVH, D), proj[:, hq + KVH * D:].view(B, KVH, D), L["k_norm"],
                       cos, sin, ring_rows, positions, self.ring_k[i], self.ring_v[i], self.ring_pos[i],
                       c.rotary_dim, c.rms_eps)
        att = ops.window_attend(q[:, None], self.ring_k[i], self.ring_v[i], self.ring_pos[i], gate=qg[..., D:])
        out = ops.linear(att.reshape(B, -1), L["w_o"], L.get("w_o@packed"), defer=True)
        if side is None:
            mo = self._memory_out(i, L, hidden, cos, sin, valid, u)
        else:
            main.wait_stream(side)
            if torch.is_tensor(mo):
                mo.record_stream(main)
        add = getattr(ops, "add_projections", None)
        return add(mo, out) if add is not None else mo + out

    def _memory_out(self, i, L, hidden, cos, sin, valid, u=None):
        """The memory path and its output projection (deferred: the norm after
        the layer sums it with the attention output projection)."""
        read = self._memory_path(i, L, hidden, cos, sin, valid, u)
        return self.ops.linear(read.reshape(read.shape[0], -1), L["m_o"], L.get("m_o@packed"), defer=True)

    def _memory_path(self, i, L, hidden, cos, sin, valid, u=None):
        """Anchor-memory read (gated) and commit of one decode token per slot."""
        c, ops = self.cfg, self.ops
        mq, mgate, mk, mv, mscores = self._memory_decode(L, hidden, cos, sin, u)
        read = ops.memory_read(mq[:, None], self.memory[i], valid=valid, head_gate=mgate)
        ops.memory_commit(mk[:, None], mv[:, None], mscores[:, None], valid, c.memory_chunk, self.memory[i])
        return read

    def _side_stream(self, x):
        if not (getattr(self, "overlap", False) and x.is_cuda):
            return None
        if getattr(self, "_side", None) is None:
            self._side = torch.cuda.Stream(device=x.device)   # default priority
        return self._side

    def decode_step(self, tokens, positions, valid=None, float_logits=True, finished=None, slot_rows=None):
        """One token for every slot: tokens, positions [B] int64, valid [B]
        bool (or None: ~finished & (slot_rows >= 0) from those [B] tensors)
        -> logits [B, V] float32 (the model dtype with ``float_logits`` off:
        the sampler widens them itself, exactly).  Updates every cache in
        place.  Each residual add is fused into the RMSNorm that follows it."""
        c, ops = self.cfg, self.ops
        h, xn, cos, sin, ring_rows, live = ops.decode_inputs(
            tokens, positions, self.embed, self.layers[0]["in_norm"], self.inv_freq, c.rms_eps,
            ring_stride=c.kv_heads * c.swa_window, window=c.swa_window,
            finished=finished if valid is None else None, slot_rows=slot_rows if valid is None else None)
        valid = live if valid is None else valid
        u = None
        for i, L in enumerate(self.layers):
            if L["kind"] == "gdn":
                delta = self._gdn_decode(i, L, xn)
            else:
                delta = self._attn_decode(i, L, xn, h, positions, cos, sin, valid, ring_rows, u)
            xn, h = ops.rmsnorm(delta, L["post_norm"], c.rms_eps, residual=h)
            nl = self.layers[i + 1] if i + 1 < len(self.layers) else None
            mlp = self._mlp(L, xn, defer=True)
            if nl is not None and nl["kind"] != "gdn":   # the memory path's own norm of the same row
                room = {"w2_row": c.hidden + c.writer_intermediate} if "m_kv@fused" in nl else {}
                xn, h, u = ops.rmsnorm(mlp, nl["in_norm"], c.rms_eps, residual=h, w2=nl["m_in_norm"], **room)
            else:
                xn, h = ops.rmsnorm(mlp, self.final_norm if nl is None else nl["in_norm"], c.rms_eps, residual=h)
        logits = ops.linear(xn, self.lm_head, self.lm_head_packed)
        return logits.float() if float_logits else logits

    # ---------------- prefill ----------------
    def prefill(self, prompts, *, token_chunk=16384, max_tokens=1 << 17):
        """Prefill fresh sequences from empty caches.

        ``prompts``: [R, T] int64, or a list of R 1-D int64 token tensors of
        any lengths (>= 1 each).  The prompts are packed into one token stream
        (cu_seqlens) and every layer runs once over it: one conv, one GDN
        chunk launch and one window-attention launch per layer for the whole
        ragged set.  A prompt longer than a piece (``token_chunk`` tokens, and
        at most ``max_tokens`` packed tokens per pass) is taken in pieces, each
        continuing the caches the previous one left: the GDN state as the
        chunk kernel's initial state, the conv window, the SWA ring as the
        window's left context, the anchor memory through _sequence with a
        state -- the reference's token-chunked prefill (runtime/model/
        inference_kernels.py:1246-1270; modeling_yanchor.py:981-1012).
        Positions start at 0 for every prompt (the logical positions of a
        left-padded batch, inference_kernels.py:1245).

        Returns (logits of each prompt's last token [R, V] float32, caches of
        [R, ...] tensors in cache_tensors() order)."""
        c, dev = self.cfg, self.device
        seqs = list(prompts.unbind(0)) if torch.is_tensor(prompts) and prompts.ndim == 2 else list(prompts)
        seqs = [torch.as_tensor(x).reshape(-1).to(torch.long) for x in seqs]
        if not seqs:
            raise ValueError("prefill needs at least one prompt")
        lengths = [int(x.numel()) for x in seqs]
        if min(lengths) < 1:
            raise ValueError("prompts must hold at least one token")
        r = len(seqs)
        piece = max(1, min(int(token_chunk), int(max_tokens) // r))
        tmp = Model.__new__(Model)
        tmp.cfg, tmp.B, tmp.device, tmp.dtype, tmp.ops, tmp.layers = c, r, dev, self.dtype, self.ops, self.layers
        tmp.state_dtype = self.state_dtype
        tmp._alloc_caches()
        last = torch.empty(r, c.hidden, dtype=self.dtype, device=dev)
        for w0 in range(0, max(lengths), piece):
            starts = [min(w0, n) for n in lengths]
            lens = [max(0, min(piece, n - w0)) for n in lengths]
            toks = torch.cat([x[w0: w0 + n] for x, n in zip(seqs, lens) if n]).to(dev)
            h = self._prefill_piece(tmp, toks, starts, lens)
            ends = [i for i, n in enumerate(lengths) if w0 < n <= w0 + piece]
            if ends:
                off = [0]
                for n in lens:
                    off.append(off[-1] + n)
                src = torch.tensor([off[i] + lens[i] - 1 for i in ends], device=dev)
                last.index_copy_(0, torch.tensor(ends, device=dev), h.index_select(0, src))
        xn = self.ops.rmsnorm(last, self.final_norm, c.rms_eps)
        logits = F.linear(xn, self.lm_head).float()
        return logits, tmp.cache_tensors()

    def _prefill_piece(self, tmp, tokens, starts, lens):
        """One pass of the layers over packed pieces: tokens [N] (the pieces
        in row order), starts / lens host ints per row of ``tmp`` (lens may
        be 0).  Updates tmp's caches in place; returns the last layer's
        residual stream [N, hidden]."""
        c, dev, ops = self.cfg, self.device, self.ops
        off = [0]
        for n in lens:
            off.append(off[-1] + n)
        cu = torch.tensor(off, dtype=torch.int32, device=dev)
        pos = torch.cat([torch.arange(s, s + n) for s, n in zip(starts, lens)]).to(dev)
        starts_t = torch.tensor(starts, dtype=torch.int64, device=dev)
        cos, sin = rope_tables(pos, c)
        h = self.embed[tokens]
        for i, L in enumerate(self.layers):
            xn = ops.rmsnorm(h, L["in_norm"], c.rms_eps)
            if L["kind"] == "gdn":
                delta = self._gdn_prefill(i, L, tmp, xn, cu, lens)
            else:
                delta = self._attn_prefill(i, L, tmp, xn, h, cos, sin, cu, starts_t, lens)
            h = h + delta
            h = h + self._mlp(L, ops.rmsnorm(h, L["post_norm"], c.rms_eps))
        return h

    def _gdn_prefill(self, i, L, tmp, xn, cu, lens):
        """GDN mixer over packed pieces: conv (continuing the window), the
        chunked recurrence from the state each row holds (one launch for all
        rows), the gated norm and the output projection."""
        c, ops = self.cfg, self.ops
        n = xn.shape[0]
        hk, dk, hv, dv = c.gdn_heads_k, c.gdn_dk, c.gdn_heads_v, c.gdn_dv
        proj = F.linear(xn, L["w_in"])                                      # [N, qkv | z | b | a]
        mixed = ops.conv_prefill(proj, tmp.conv_state[i], L["conv_w"], cu, c.conv_dim, lens)
        _, _, beta, g = self._gdn_split(L, proj)
        q = mixed[:, : hk * dk].reshape(1, n, hk, dk)
        k = mixed[:, hk * dk: 2 * hk * dk].reshape(1, n, hk, dk)
        v = mixed[:, 2 * hk * dk:].reshape(1, n, hv, dv)
        # the chunked recurrence runs from and to float32; a float16 store rounds once a piece
        o, st = ops.gdn_prefill(q, k, v, g[None], beta[None], cu, lens, initial_state=tmp.gdn_state[i].float())
        tmp.gdn_state[i].copy_(st)
        y = ops.gated_rmsnorm(o.reshape(n, hv, dv), proj[:, c.conv_dim: c.conv_dim + hv * dv], L["gnorm"],
                              c.rms_eps)
        return F.linear(y, L["w_out"])

    def _attn_prefill(self, i, L, tmp, xn, hidden, cos, sin, cu, starts, lens):
        """SWA + anchor-memory mixer over packed pieces: the window attention
        reads each row's ring as left context, the pieces' keys then fill the
        ring; the memory reads and writes through _sequence with the row's
        state."""
        c, ops = self.cfg, self.ops
        n = xn.shape[0]
        H, G, D = c.attn_heads, c.kv_heads, c.head_dim
        proj = F.linear(xn, L["w_qkv"])                                     # [N, (q|gate) per head | k | v]
        hq = 2 * H * D
        qg = proj[:, :hq].view(n, H, 2 * D)
        q = ops.head_norm_rope(qg[..., :D], L["q_norm"], cos, sin, c.rotary_dim, c.rms_eps)
        k = ops.head_norm_rope(proj[:, hq: hq + G * D].view(n, G, D), L["k_norm"], cos, sin, c.rotary_dim,
                               c.rms_eps)
        v = proj[:, hq + G * D:].view(n, G, D)
        rows = torch.arange(len(lens), device=xn.device)
        att = ops.swa_prefill(q, k, v, cu, starts, tmp.ring_k[i], tmp.ring_v[i], rows, gate=qg[..., D:],
                              lengths=lens)
        ops.ring_fill(k, v, cu, starts, rows, tmp.ring_k[i], tmp.ring_v[i], tmp.ring_pos[i], lengths=lens)
        out = F.linear(att.reshape(n, H * D), L["w_o"])
        u = ops.rmsnorm(hidden, L["m_in_norm"], c.rms_eps)
        mq, mgate, mk, mv, msc = self._memory_decode(L, hidden, cos, sin, u)
        read = self._memory_prefill(tmp.memory[i], mq, mk, mv, msc, lens)
        return out + F.linear((read * mgate[..., None].to(read.dtype)).reshape(n, H * D), L["m_o"])

    def _memory_prefill(self, state, q, key, value, scores, lens):
        """_sequence over packed pieces: the rows with tokens are laid out as
        a right-padded [R', Lmax] batch (padding invalid, which _sequence's
        stable argsort takes as absent) on their own state rows; returns the
        read of every packed token [N, H, D]."""
        c, dev = self.cfg, q.device
        live = [r for r, n in enumerate(lens) if n]
        nl = [lens[r] for r in live]
        lmax = max(nl)
        if len(live) == len(lens) and min(nl) == lmax:
            b = len(live)
            read = self.ops.memory_sequence(q.view(b, lmax, *q.shape[1:]), key.view(b, lmax, *key.shape[1:]),
                                            value.reshape(b, lmax, *value.shape[1:]).contiguous(),
                                            scores.view(b, lmax, -1).float(), None, c.memory_chunk, state)
            return read.reshape(q.shape)
        bi = torch.repeat_interleave(torch.arange(len(live), device=dev), torch.tensor(nl, device=dev))
        ti = torch.cat([torch.arange(n, device=dev) for n in nl])

        def pad(x, fill=0.0):
            out = torch.full((len(live), lmax) + tuple(x.shape[1:]), fill, dtype=x.dtype, device=dev)
            out[bi, ti] = x
            return out

        valid = pad(torch.ones(q.shape[0], dtype=torch.bool, device=dev), False)
        rows = torch.tensor(live, device=dev)
        sub = state if len(live) == len(lens) else state.select(rows)
        read = self.ops.memory_sequence(pad(q), pad(key), pad(value.contiguous()), pad(scores.float()), valid,
                                        c.memory_chunk, sub)
        if sub is not state:
            state.scatter_(sub, rows, torch.arange(len(live), device=dev))
        return read[bi, ti]


@dataclass
class Request:
    attempt_id: int
    prompt: torch.Tensor
    cap: int
    arrival_step: int
    row: int = -1                 # storage row, set at admission
    group: int | None = None      # prefill group: requests of one group share one prompt and one prefill

    @property
    def group_id(self):
        """The prefill group id, the attempt id when none is set (as
        runtime/inference.py:92 defaults it)."""
        return self.attempt_id if self.group is None else int(self.group)


# The mechanical-repetition stop (reference runtime/scoring/protocols.py:73-76):
# a tail of REPEAT_COUNT exact repeats of a period in [MIN, MAX] tokens.
REPEAT_MIN_PERIOD, REPEAT_MAX_PERIOD, REPEAT_COUNT = 128, 256, 8


def repetition_periods(tails, lengths, min_period=REPEAT_MIN_PERIOD, max_period=REPEAT_MAX_PERIOD,
                       repeats=REPEAT_COUNT):
    """For each row of ``tails`` [N, W] (a sequence's last W tokens, the
    valid ones right-aligned: ``lengths`` [N] of them), the smallest period P
    in [min_period, max_period] such that the last repeats * P valid tokens
    are ``repeats`` copies of one P-token block, else 0
    (mechanical_repetition_early_stop_patterns, runtime/scoring/protocols.py:
    89-109)."""
    import numpy as np
    tails = np.asarray(tails)
    lengths = np.minimum(np.asarray(lengths), tails.shape[1])
    out = np.zeros(len(tails), dtype=np.int32)
    top = min(max_period, tails.shape[1] // repeats)
    for i in range(len(tails)):
        for period in range(min_period, top + 1):
            if lengths[i] < period * repeats:
                break
            block = tails[i, tails.shape[1] - period * repeats:].reshape(repeats, period)
            if (block == block[-1]).all():
                out[i] = period
                break
    return out


@dataclass
class EngineMetrics:
    decode_useful_token_events: int = 0
    decode_scheduled_token_events: int = 0
    decode_steps: int = 0
    generation_wall_seconds: float = 0.0
    initial_prefill_seconds: float = 0.0
    refill_prefill_seconds: float = 0.0
    refilled: int = 0
    completed: int = 0
    peak_allocated_gib: float = 0.0
    extra: dict = field(default_factory=dict)

    @property
    def decode_seconds(self):
        return self.generation_wall_seconds - self.initial_prefill_seconds - self.refill_prefill_seconds

    @property
    def decode_tokens_per_second(self):
        return self.decode_useful_token_events / max(self.decode_seconds, 1e-9)


class Engine:
    """Continuous-batching decode driver over ``Model`` (the synthetic-request
    counterpart of cuda_graph_generate_top20_dynamic_refill,
    runtime/model/inference_kernels.py:1351-1765).

    Slots are a fixed physical batch; every decode step computes all of them
    (finished / empty slots are scheduled but not useful, as in the reference).
    At poll points (every ``poll_interval`` steps, a host sync) finished slots
    are refilled from the arrival queue in ascending slot order: the new
    requests are prefilled together and their caches scattered into the slots.
    The decode step -- model forward, top-k/top-p counter sampling with the
    presence penalty fused, slot bookkeeping -- is one captured HIP graph.
    """

    def __init__(self, model: Model, *, seed=20260923, temperature=0.6, top_k=20, top_p=0.95,
                 presence_penalty=1.5, poll_interval=32, max_rows=4096, max_new_tokens=8192, use_graph=True,
                 tail_compaction=False, tail_compaction_live_fraction=0.5, eos_token_ids=(), pad_token_id=0,
                 sampling_backend="triton_top20", mechanical=False, prefill_tokens=1 << 17):
        """``sampling_backend``: "triton_top20" (the fused top-k kernel's
        semantics) or "torch" (sample_top_k_top_p_counter's, every top_k);
        ``eos_token_ids``: at most two ids that finish a sequence;
        ``mechanical``: stop a sequence whose tail repeats mechanically
        (checked at poll points, as the reference); ``prefill_tokens``: prompt
        tokens per packed prefill of an admission."""
        if len(eos_token_ids) > 2:
            raise ValueError("the decode bookkeeping takes at most two EOS ids")
        if sampling_backend not in ("triton_top20", "torch"):
            raise ValueError("counter sampling backend must be torch or triton_top20")
        self.m, self.B, self.dev = model, model.B, model.device
        self.eos, self.pad, self.sampling_backend = tuple(int(x) for x in eos_token_ids), int(pad_token_id), \
            sampling_backend
        self.mechanical = mechanical
        self.seed, self.temperature, self.top_k, self.top_p = seed, temperature, top_k, top_p
        self.penalty, self.poll_interval, self.use_graph = presence_penalty, poll_interval, use_graph
        self.tail_compaction, self.tail_fraction = tail_compaction, tail_compaction_live_fraction
        self.compactions: list = []
        self.max_rows, self.max_new = max_rows, max_new_tokens
        B, dev, V = self.B, self.dev, model.cfg.vocab
        self.decode_ids = torch.zeros(B, 1, dtype=torch.long, device=dev)
        self.positions = torch.zeros(B, dtype=torch.long, device=dev)
        self.finished = torch.ones(B, dtype=torch.bool, device=dev)
        self.slot_rows = torch.full((B,), -1, dtype=torch.long, device=dev)
        self.slot_caps = torch.zeros(B, dtype=torch.long, device=dev)
        self.row_steps = torch.ones(B, dtype=torch.long, device=dev)
        self.attempt_ids = torch.zeros(B, dtype=torch.long, device=dev)
        self.dense_seen = torch.zeros(B, V, dtype=torch.bool, device=dev)
        self.storage = torch.zeros(max_rows + B, max_new_tokens + 1, dtype=torch.int32, device=dev)
        self.generated = torch.zeros(max_rows + B, dtype=torch.long, device=dev)
        self.finished_by_eos = torch.zeros(max_rows + B, dtype=torch.bool, device=dev)
        self.finished_by_repetition: set = set()      # storage rows stopped by the repetition check
        self.sink_rows = max_rows + torch.arange(B, device=dev)
        self.useful = torch.zeros((), dtype=torch.long, device=dev)
        self.graph = None
        self.next_row = 0
        self.slot_request: list = [None] * B
        self.row_request: dict = {}          # storage row -> the request it holds (the latest one)
        self.prefill_tokens = int(prefill_tokens)
        self.prefill_calls = 0               # Model.prefill calls (one packed prefill each)
        self.prefill_unique_rows = self.prefill_expanded_rows = 0
        self.live_capture_steps = 0          # decode steps run by live re-captures (after compaction)

    # one decode step on the device (captured)
    def _step(self):
        logits = self.m.decode_step(self.decode_ids[:, 0], self.positions, float_logits=False,
                                    finished=self.finished, slot_rows=self.slot_rows)
        tok = self.m.ops.sample(logits, self.attempt_ids, self.row_steps, self.dense_seen, seed=self.seed,
                                temperature=self.temperature, top_k=self.top_k, top_p=self.top_p,
                                penalty=self.penalty, backend=self.sampling_backend)
        self.m.ops.bookkeeping(tok, self.storage, self.dense_seen, self.generated, self.finished_by_eos,
                               self.finished, self.slot_rows, self.sink_rows, self.slot_caps, self.row_steps,
                               self.positions, self.decode_ids, self.useful,
                               maximum_new_tokens=self.max_new, pad_token_id=self.pad, eos_token_ids=self.eos)

    CAPTURE_WARMUP = 2

    def capture(self, live=False):
        """Warm up and capture the decode step; returns the number of eager
        warm-up steps run (0 when nothing is captured).  They are ordinary
        decode steps: call with every slot empty (they then only touch rows
        that admission overwrites whole), or with ``live`` set when live slots
        may take them as real steps (after compaction)."""
        if not self.use_graph or self.graph is not None:
            return 0
        if not live and bool(((~self.finished) & (self.slot_rows >= 0)).any()):
            raise RuntimeError("capture() with live slots would advance them; pass live=True to allow it")
        for _ in range(self.CAPTURE_WARMUP):  # warm the allocator and the sampler workspace outside capture
            self._step()
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._step()
        torch.cuda.synchronize()
        return self.CAPTURE_WARMUP

    def step(self):
        if self.use_graph:
            if self.graph is None:
                raise RuntimeError("Engine.capture() must run before the first admission")
            self.graph.replay()
        else:
            self._step()

    def admit(self, requests, targets, rows=None):
        """Prefill ``requests`` and place them in slots ``targets`` (host
        lists), their tokens in storage ``rows`` (default: the next free
        rows).  Requests of one prefill group (``Request.group``) must hold
        the same prompt; each group is prefilled once and its caches copied
        to every member's slot (build_prefill_expansion /
        assert_group_rows_identical, runtime/model/inference_kernels.py:
        90-121, 1226-1238).  The distinct prompts, of any lengths, are packed
        into one prefill (one GDN chunk launch per layer) per
        ``prefill_tokens`` of prompt.  Returns the prefill seconds."""
        if not requests:
            return 0.0
        from . import inference_kernels as ik
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        n = len(requests)
        if rows is None:
            rows = list(range(self.next_row, self.next_row + n))
            self.next_row += n
        if max(rows) >= self.max_rows:
            raise ValueError(f"storage row {max(rows)} past the engine's {self.max_rows} rows")
        reps, inverse, seen = [], [], {}
        for j, r in enumerate(requests):
            u = seen.get(r.group_id)
            if u is None:
                seen[r.group_id] = u = len(reps)
                reps.append(j)
            elif not torch.equal(requests[reps[u]].prompt, r.prompt):
                raise ValueError("prefill group contains non-identical rows")
            inverse.append(u)
        batches, cur, tokens = [], [], 0
        for u, j in enumerate(reps):
            length = int(requests[j].prompt.numel())
            if cur and tokens + length > self.prefill_tokens:
                batches.append(cur)
                cur, tokens = [], 0
            cur.append(u)
            tokens += length
        batches.append(cur)
        for batch in batches:
            place = {u: i for i, u in enumerate(batch)}
            members = [j for j in range(n) if inverse[j] in place]
            logits, caches = self.m.prefill([requests[reps[u]].prompt for u in batch])
            self.prefill_calls += 1
            src = torch.tensor([place[inverse[j]] for j in members], dtype=torch.long, device=self.dev)
            ids = torch.tensor([requests[j].attempt_id for j in members], dtype=torch.long, device=self.dev)
            first = self.m.ops.sample(logits.index_select(0, src), ids, 0, None, seed=self.seed,
                                      temperature=self.temperature, top_k=self.top_k, top_p=self.top_p,
                                      penalty=0.0, backend=self.sampling_backend)
            tgt = torch.tensor([targets[j] for j in members], dtype=torch.long, device=self.dev)
            ik.gather_rows(list(zip(caches, self.m.cache_tensors())), src, tgt, len(members))
            del caches
            rws = torch.tensor([rows[j] for j in members], dtype=torch.long, device=self.dev)
            caps = torch.tensor([requests[j].cap for j in members], dtype=torch.long, device=self.dev)
            lens = torch.tensor([int(requests[j].prompt.numel()) for j in members], dtype=torch.long,
                                device=self.dev)
            is_eos = torch.zeros(len(members), dtype=torch.bool, device=self.dev)
            for e in self.eos:
                is_eos |= first[:, 0] == e
            done = (caps <= 1) | is_eos
            self.slot_rows.index_copy_(0, tgt, rws)
            self.slot_caps.index_copy_(0, tgt, caps)
            self.attempt_ids.index_copy_(0, tgt, ids)
            self.row_steps.index_fill_(0, tgt, 1)
            self.positions.index_copy_(0, tgt, lens)
            self.finished.index_copy_(0, tgt, done)
            self.decode_ids.index_copy_(0, tgt, torch.where(done[:, None], torch.full_like(first, self.pad), first))
            self.dense_seen.index_fill_(0, tgt, False)
            self.dense_seen[tgt, first[:, 0]] = True
            self.storage[rws, 0] = first[:, 0].to(torch.int32)
            self.generated[rws] = 1
            self.finished_by_eos[rws] = is_eos
        for r, s_, w in zip(requests, targets, rows):
            self.slot_request[s_] = r
            r.row = w
            self.finished_by_repetition.discard(w)
            self.row_request[w] = r
        self.prefill_unique_rows += len(reps)
        self.prefill_expanded_rows += n
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    def check_repetition(self):
        """The reference's mechanical-repetition stop at a poll point
        (runtime/model/inference_kernels.py:1518-1539): live slots with at
        least 8 x 128 tokens whose tail is 8 exact repeats of a period in
        [128, 256] are finished.  Returns the number stopped (a host sync)."""
        live = ((~self.finished) & (self.slot_rows >= 0) & (self.row_steps >= REPEAT_MIN_PERIOD * REPEAT_COUNT))
        slots = torch.nonzero(live).flatten()
        if not slots.numel():
            return 0
        rows = self.slot_rows[slots]
        lengths = self.row_steps[slots]
        width = REPEAT_MAX_PERIOD * REPEAT_COUNT
        rel = torch.arange(-width, 0, device=self.dev)[None]
        pos = lengths[:, None] + rel
        tails = self.storage[rows[:, None], pos.clamp_min(0)].cpu().numpy()
        periods = repetition_periods(tails, torch.clamp(lengths, max=width).cpu().numpy())
        stop = [int(s_) for s_, p in zip(slots.tolist(), periods) if p]
        for s_, p in zip(slots.tolist(), periods):
            if p:
                self.finished_by_repetition.add(int(self.slot_rows[s_]))
        if stop:
            self.finished[torch.tensor(stop, device=self.dev)] = True
        return len(stop)

    def fill(self, queue):
        """Initial fill of the physical batch (runtime/model/inference_kernels.py:
        1386-1450): the queued attempts are ordered by ``_initial_attempt_order``
        (largest cap first, then attempt id), the first ``B`` of them are
        prefilled together into slots 0..B-1 and the rest stay queued in that
        order.  Returns the prefill seconds (excluded from decode time, as the
        reference's initial prefill)."""
        from . import inference_kernels as ik
        if not queue:
            return 0.0
        groups = [r.group_id for r in queue]
        order = ik._initial_attempt_order([r.cap for r in queue], [r.attempt_id for r in queue], groups)
        take = min(self.B, len(queue), self.max_rows - self.next_row)
        if take < len(queue) and ik._group_aligned_prefix_length(order, groups, take) != take:
            raise ValueError("slot batch size splits a repeated-prompt prefill group")
        first = [queue[i] for i in order[:take]]
        queue[:] = [queue[i] for i in order[take:]]
        return self.admit(first, list(range(take)))

    def outputs(self):
        """{attempt id: generated token ids} of the request each storage row
        holds (its latest admission; a host sync)."""
        rows = sorted(self.row_request)
        if not rows:
            return {}
        idx = torch.tensor(rows, dtype=torch.long, device=self.dev)
        lengths = self.generated.index_select(0, idx).tolist()
        data = self.storage.index_select(0, idx).cpu()
        return {self.row_request[w].attempt_id: data[i, : lengths[i]].tolist() for i, w in enumerate(rows)}

    def live_slots(self):
        """Slots that run a sequence this step (a host sync)."""
        return int(((~self.finished) & (self.slot_rows >= 0)).sum())

    def poll(self, queue, exhausted=False):
        """Host sync: refill finished slots (ascending) from the queue; with
        tail compaction on and no more arrivals (``exhausted``), shrink the
        physical batch once few slots are live."""
        if self.mechanical:
            self.check_repetition()
        fin = self.finished.cpu().tolist()
        free = [s for s, f in enumerate(fin) if f]
        completed = sum(1 for s in free if self.slot_request[s] is not None)
        for s in free:
            self.slot_request[s] = None
        take = min(len(free), len(queue), self.max_rows - self.next_row)
        reqs = [queue.pop(0) for _ in range(take)]
        t = self.admit(reqs, free[:take])
        empty = torch.tensor(free[take:], dtype=torch.long, device=self.dev)
        if empty.numel():
            self.slot_rows.index_fill_(0, empty, -1)
            self.finished.index_fill_(0, empty, True)
        live = self.B - len(free) + take
        if self.tail_compaction and self.B > 1 and exhausted and not queue and \
                0 < live < self.B and live <= max(1, int(self.B * self.tail_fraction)):
            self.live_capture_steps += self.compact()
        return t, completed, take

    def compact(self):
        """Tail compaction (runtime/model/inference_kernels.py:1724-1745): keep
        the live slots in ascending order, gather their cache rows into a
        smaller physical batch in one launch, and capture the decode step
        again.  The capture's eager warm-up steps are real decode steps of the
        live slots (bookkeeping counts them), as the reference's
        consume_capture_steps; returns their number."""
        from . import inference_kernels as ik
        keep = ik.compaction_keep(self.finished, self.slot_rows)
        n = int(keep.numel())
        if n == 0 or n == self.B:
            return 0
        torch.cuda.synchronize()
        self.graph = None
        old = self.m.cache_tensors()
        self.m.B = n
        self.m._alloc_caches()
        ik.gather_rows(list(zip(old, self.m.cache_tensors())), keep, None, n)
        del old
        for name in ("decode_ids", "positions", "finished", "slot_rows", "slot_caps", "row_steps", "attempt_ids",
                     "dense_seen"):
            setattr(self, name, getattr(self, name).index_select(0, keep))
        self.slot_request = [self.slot_request[i] for i in keep.tolist()]
        self.B = n
        self.sink_rows = self.max_rows + torch.arange(n, device=self.dev)
        self.compactions.append(n)
        return self.capture(live=True)


def synthetic_requests(steps, *, rate=4.0, prompt_len=128, mean_len=1024, max_len=8192, vocab=151936,
                       seed=20260923, initial=0):
    """``initial`` requests queued before step 0 (the backlog that fills the
    physical batch), then Poisson(rate) arrivals per step; uniform-random
    prompts and geometric(mean_len) generation lengths (capped at max_len)."""
    gen = torch.Generator().manual_seed(seed)
    arrivals = torch.poisson(torch.full((steps,), float(rate)), generator=gen).long().tolist()
    if arrivals:
        arrivals[0] += int(initial)
    reqs, aid = [], 0
    p = 1.0 / mean_len
    for step, n in enumerate(arrivals):
        for _ in range(n):
            u = torch.rand((), generator=gen).item()
            length = min(max_len, max(1, int(math.ceil(math.log1p(-u) / math.log1p(-p)))))
            prompt = torch.randint(0, vocab, (prompt_len,), generator=gen)
            reqs.append(Request(aid, prompt, length, step))
            aid += 1
    return reqs


def run_decode_benchmark(model: Model, *, steps, warmup, rate=4.0, prompt_len=128, mean_len=1024,
                         poll_interval=32, seed=20260923, use_graph=True, max_new_tokens=8192, requests=None,
                         tail_compaction=False, engine=None, initial_fill=True, progress_every=0):
    """Continuous batching for warmup + steps decode steps; returns metrics of
    the timed steps (the reference's decode tokens/s definition).

    Arrivals are ``synthetic_requests`` (a backlog of one request per slot
    before step 0, then Poisson(rate) per step) unless ``requests`` is given.
    With ``initial_fill`` the requests queued at step 0 fill the physical
    batch before the first step (``Engine.fill``, the reference's initial
    prefill); later arrivals refill finished slots at the poll points.  The
    live slots of every timed step are recorded (``extra["live_slots"]``:
    min / mean / first / last) from the device's useful-event counter, one
    8-byte device copy per step."""
    eng = engine or Engine(model, seed=seed, poll_interval=poll_interval, use_graph=use_graph,
                           max_new_tokens=max_new_tokens, tail_compaction=tail_compaction)
    eng.capture()
    if requests is None:
        requests = synthetic_requests(warmup + steps, rate=rate, prompt_len=prompt_len, mean_len=mean_len,
                                      max_len=max_new_tokens, vocab=model.cfg.vocab, seed=seed,
                                      initial=eng.B if initial_fill else 0)
    queue, pending, idx = [], sorted(requests, key=lambda r: r.arrival_step), 0
    m = EngineMetrics()
    total = warmup + steps
    t_start = None
    useful0 = 0
    hist = torch.zeros(steps + 1, dtype=torch.long, device=eng.dev)
    # per timed step, the slots' positions and live flags as the step reads
    # them (two small device copies a step), for the SWA rings' live fraction
    pos_hist = torch.zeros(steps, eng.B, dtype=torch.long, device=eng.dev)
    live_hist = torch.zeros(steps, eng.B, dtype=torch.bool, device=eng.dev)
    fill_seconds = 0.0
    for step in range(total):
        while idx < len(pending) and pending[idx].arrival_step <= step:
            queue.append(pending[idx])
            idx += 1
        if step == 0 and initial_fill:
            fill_seconds = eng.fill(queue)      # before the timed window: not part of its wall time
        if step == warmup and warmup % poll_interval and initial_fill:
            eng.poll(queue, exhausted=idx >= len(pending))   # the timed window starts with every slot live
        if step == warmup:
            torch.cuda.synchronize()
            hist[0].copy_(eng.useful)
            useful0 = int(eng.useful.item())
            t_start = time.perf_counter()
            m.refill_prefill_seconds = 0.0
        if step % poll_interval == 0:
            live_steps = eng.live_capture_steps
            t, done, taken = eng.poll(queue, exhausted=idx >= len(pending))
            if t_start is not None:
                m.refill_prefill_seconds += t
                m.refilled += taken
                m.completed += done
                # a compaction's re-capture ran real decode steps of the live slots
                m.decode_scheduled_token_events += (eng.live_capture_steps - live_steps) * eng.B
        if t_start is not None and eng.B == pos_hist.shape[1]:
            pos_hist[m.decode_steps].copy_(eng.positions)
            torch.logical_not(eng.finished, out=live_hist[m.decode_steps])
        eng.step()
        if progress_every and (step + 1) % progress_every == 0:
            print(f"[decode] step {step + 1} of {total} enqueued", flush=True)
        if t_start is not None:
            m.decode_steps += 1
            m.decode_scheduled_token_events += eng.B
            hist[m.decode_steps].copy_(eng.useful)
    torch.cuda.synchronize()
    m.generation_wall_seconds = time.perf_counter() - t_start
    m.decode_useful_token_events = int(eng.useful.item()) - useful0
    m.peak_allocated_gib = torch.cuda.max_memory_allocated() / 2**30
    live = (hist[1:] - hist[:-1]).cpu()
    # a step at position p reads min(p + 1, W) live ring slots (its own token
    # is written before the read); averaged over the live slots of the timed
    # steps recorded at full width
    window = model.cfg.swa_window
    lh = live_hist[: m.decode_steps]
    fill = (pos_hist[: m.decode_steps] + 1).clamp(max=window).float() / window
    ring_fill = float((fill * lh).sum() / lh.sum().clamp(min=1))
    m.extra = {"queue_left": len(queue), "live_slots_end": eng.live_slots(), "ring_fill": ring_fill,
               "live_slots": {"min": int(live.min()), "mean": float(live.float().mean()),
                              "first": int(live[0]), "last": int(live[-1])} if steps else {},
               "physical_slots": eng.B, "tail_compactions": list(eng.compactions),
               "initial_prefill_seconds": fill_seconds}
    return m
