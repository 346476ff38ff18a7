"""The decode step's ops on the host, from the oracle's restatements only
(oracle; test infrastructure: imported by tests/ and by bench.py's CPU
baseline leg, never by the product).

``HostOps`` implements the ops interface that ``yanchor_amd.runtime.Model``
calls for one decode token per slot (and the two a prefill calls), so the
product's model wiring can run on the CPU in float32 with every piece of
arithmetic of the decode step taken from ``oracle/``:

* the GDN recurrence          ``oracle.gdn.recurrent_gated_delta_rule``
                              (wheel transformers/models/qwen3_5/
                              modeling_qwen3_5.py:314-353) and, for prefill,
                              its chunked form per packed sequence (234-311);
* the anchor memory           ``oracle.anchor.committed_read`` /
                              ``commit_decode`` (modeling_yanchor.py:283-312)
                              and, for prefill, ``sequence`` (178-275);
* the SWA ring read / write   ``oracle.glue.ring_decode_attention``
                              (runtime/model/inference_kernels.py:1881-1898) and
                              the chronological ring write (1828-1856);
* the layer glue              ``oracle.glue``: Qwen3_5RMSNorm, the gated
                              norm, the conv update of the CUDA backend, the
                              gates, RoPE, the memory's query side
                              (modeling_yanchor.py:168-176) and the writer's
                              silu * up (147-166);
* sampling and bookkeeping    ``oracle.sampling`` / ``oracle.slots``.

Arguments and results follow the runtime's ops (the same names, layouts and
return tuples); tensors are float32 on the host.

``BatchedHostOps`` is the same with the anchor read and commit over the whole
batch at once (``committed_read_batched`` / ``commit_decode_batched``, the
reference's torch branch, pinned equal to the per-row forms): the host CPU
baseline's ops.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from oracle import anchor, gdn, glue, sampling, slots

HEAD_DIM = 128


def gate_read(read, valid=None, head_gate=None):
    """The decode layer's gating of a memory read [B, 1, H, D]:
    read * valid (modeling_yanchor.py:313) times the per-head read gate of
    _query_scores (modeling_yanchor.py:170, applied at 316)."""
    if valid is not None:
        read = read * valid[:, None, None, None].to(read.dtype)
    if head_gate is not None:
        read = read * head_gate[:, None, :, None].to(read.dtype)
    return read


class HostOps:
    """The runtime's decode ops on the CPU from the oracle's functions."""

    # ---- layer glue ----
    @staticmethod
    def decode_inputs(tokens, positions, embed, w, inv_freq, eps, *, ring_stride, window, finished=None,
                      slot_rows=None):
        """Embedding row, the first layer's input norm, the rotary tables
        (rope_cos_sin), the SWA ring row b * ring_stride + position % window
        and the live-slot mask ~finished & slot_rows >= 0."""
        h = embed[tokens]
        cos, sin = glue.rope_cos_sin(positions, inv_freq, torch.float32)
        rows = torch.arange(tokens.shape[0]) * ring_stride + positions % window
        valid = None if finished is None else (~finished) & (slot_rows >= 0)
        return h, glue.rms_norm(h, w, eps), cos, sin, rows, valid

    @staticmethod
    def rmsnorm(x, w, eps, residual=None, w2=None):
        """Qwen3_5RMSNorm of x (+ residual); returns the normed row, then the
        sum when a residual is given, then the row normed with w2."""
        s = x if residual is None else x + residual
        out = [glue.rms_norm(s, w, eps)]
        if residual is not None:
            out.append(s)
        if w2 is not None:
            out.append(glue.rms_norm(s, w2, eps))
        return out[0] if len(out) == 1 else tuple(out)

    @staticmethod
    def linear(x, w, packed=None, residual=None, defer=False):
        out = F.linear(x, w)
        return out if residual is None else out + residual

    @staticmethod
    def silu_mul(gate_up):
        gate, up = gate_up.chunk(2, -1)
        return glue.silu_mul(gate, up)

    def mlp_act(self, x, w, packed=None):
        return self.silu_mul(F.linear(x, w))

    @staticmethod
    def gdn_prep(proj, conv_state, conv_w, a_log, dt_bias, *, conv_dim, qk_dim, hv, b_offset, a_offset):
        """Conv update of the CUDA backend (the runtime's conv window is
        time-major [B, K-1, C]; the oracle's state is [B, C, K-1]) and the
        gates; returns q, k, v, g, beta."""
        st = conv_state.transpose(1, 2).contiguous()
        mixed = glue.causal_conv1d_update_cuda(proj[:, :conv_dim, None], st, conv_w)[..., 0]
        conv_state.copy_(st.transpose(1, 2))
        beta, g = glue.gdn_gates(proj[:, b_offset: b_offset + hv], proj[:, a_offset: a_offset + hv], a_log, dt_bias)
        return mixed[:, :qk_dim], mixed[:, qk_dim: 2 * qk_dim], mixed[:, 2 * qk_dim:], g, beta.float()

    @staticmethod
    def gated_rmsnorm(o, z, w, eps):
        b, h, d = o.shape
        return glue.gated_rms_norm(o, z.reshape(b, h, d), w, eps).reshape(b, h * d)

    @staticmethod
    def head_norm_rope(x, w, cos, sin, rotary_dim, eps):
        """Per-head Qwen3_5RMSNorm, then RoPE on the first rotary_dim dims."""
        y = glue.rms_norm(x, w, eps)
        if rotary_dim:
            y = glue.memory_rope(y, cos[:, None, :rotary_dim], sin[:, None, :rotary_dim])
        return y

    def ring_write(self, k, v, w, cos, sin, rows, positions, ring_k, ring_v, ring_pos, rotary_dim, eps):
        """The normed, rotated key, the value and the position of the decode
        token into ring slot position % window (inference_kernels.py:1828-1856)."""
        key = self.head_norm_rope(k, w, cos, sin, rotary_dim, eps)
        tok = torch.arange(k.shape[0])
        slot = positions % ring_k.shape[2]
        ring_k[tok, :, slot] = key.to(ring_k.dtype)
        ring_v[tok, :, slot] = v.to(ring_v.dtype)
        ring_pos[tok, :, slot] = positions.to(torch.int32)[:, None]

    @staticmethod
    def window_attend(q, keys, values, positions, gate=None):
        return glue.ring_decode_attention(q, keys, values, positions >= 0, gate)

    @staticmethod
    def memory_prologue(proj, heads, feat_offset, n_features, q_norm_w, cos, sin, read_scale, gate_w, gate_b,
                        adm_up, rotary_dim, eps):
        """_query_scores from the fused projection [q | features | ...]:
        q_norm, the read gate before RoPE, RoPE, the admission scores."""
        b = proj.shape[0]
        qn = glue.rms_norm(proj[:, : heads * HEAD_DIM].view(b, heads, HEAD_DIM), q_norm_w, eps)
        gate = glue.query_read_gate(qn, read_scale, gate_w, gate_b)
        q = glue.memory_rope(qn, cos[:, None, :rotary_dim], sin[:, None, :rotary_dim])
        scores = glue.admission_scores(proj[:, feat_offset: feat_offset + n_features], adm_up)
        return q, gate, scores

    # ---- the recurrence and the anchor memory ----
    @staticmethod
    def gdn_decode(q, k, v, g, beta, state):
        o, st = gdn.recurrent_gated_delta_rule(q, k, v, g, beta, state, dtype=torch.float32)
        state.copy_(st)
        return o.to(q.dtype)

    @staticmethod
    def gdn_prefill(q, k, v, g, beta, cu_seqlens, lengths, initial_state=None):
        """Packed prefill pieces from ``initial_state`` (None = zeros): the
        chunked form (wheel:234-311) per sequence of cu_seqlens; returns (o,
        final states)."""
        o, st = gdn.varlen(gdn.chunk_gated_delta_rule, q, k, v, g, beta, cu_seqlens.tolist(),
                           initial_state=initial_state, dtype=torch.float32)
        return o.to(q.dtype), st

    @staticmethod
    def conv_prefill(proj, window, conv_w, cu_seqlens, channels, lengths):
        """``glue.causal_conv1d_prefill`` per packed piece, continuing each
        row's conv window [R, 3, C] (updated in place)."""
        outs, off = [], 0
        for r, n in enumerate(lengths):
            y, new = glue.causal_conv1d_prefill(proj[off: off + n, :channels], window[r], conv_w)
            window[r].copy_(new)
            outs.append(y)
            off += n
        return torch.cat(outs)

    @staticmethod
    def _ring_context(ring, row, start, window):
        n = min(start, window - 1) if row >= 0 else 0
        slots = torch.arange(start - n, start) % window
        return ring[row][:, slots].transpose(0, 1)

    def swa_prefill(self, q, k, v, cu_seqlens, starts, ring_k, ring_v, ring_rows, gate=None, lengths=None):
        """``glue.swa_prefill_attention`` (reference_swa, modeling_yanchor.py:
        412-427) per packed piece over [the ring's entries before the piece,
        oldest first | the piece's keys], then * sigmoid(gate) with the
        sigmoid rounded to the query dtype (as ring_decode_attention)."""
        window = ring_k.shape[2]
        st, rr, cu = starts.tolist(), ring_rows.tolist(), cu_seqlens.tolist()
        out = torch.empty_like(q)
        for r in range(len(cu) - 1):
            s, e = cu[r], cu[r + 1]
            if e == s:
                continue
            kc = torch.cat((self._ring_context(ring_k, rr[r], st[r], window), k[s:e]), 0)
            vc = torch.cat((self._ring_context(ring_v, rr[r], st[r], window), v[s:e]), 0)
            nctx = kc.shape[0] - (e - s)
            for b0 in range(0, e - s, 1024):      # query blocks over the keys they can see
                b1 = min(e - s, b0 + 1024)
                lo = max(0, nctx + b0 - window + 1)
                out[s + b0: s + b1] = glue.swa_prefill_attention(
                    q[None, s + b0: s + b1], kc[None, lo: nctx + b1], vc[None, lo: nctx + b1], window,
                    query_start=nctx + b0 - lo)[0]
        if gate is not None:
            out = out * torch.sigmoid(gate.float()).to(q.dtype)
        return out

    @staticmethod
    def ring_fill(k, v, cu_seqlens, starts, ring_rows, ring_k, ring_v, ring_pos, lengths=None):
        """The chronological ring write (inference_kernels.py:1828-1856) of a
        piece's tokens in order; only the last min(window, L) survive."""
        window = ring_k.shape[2]
        st, rr, cu = starts.tolist(), ring_rows.tolist(), cu_seqlens.tolist()
        for r in range(len(cu) - 1):
            if rr[r] < 0:
                continue
            for t in range(cu[r], cu[r + 1]):
                pos = st[r] + t - cu[r]
                ring_k[rr[r], :, pos % window] = k[t].to(ring_k.dtype)
                ring_v[rr[r], :, pos % window] = v[t].to(ring_v.dtype)
                ring_pos[rr[r], :, pos % window] = pos

    @staticmethod
    def memory_sequence(q, key, value, scores, valid, chunk, state):
        """Prefill read and write continuing ``state`` (_sequence,
        modeling_yanchor.py:178-275)."""
        return anchor.sequence(q, key, value, scores, valid, chunk, state, dtype=torch.float32).to(q.dtype)

    @staticmethod
    def memory_read(q, state, valid=None, head_gate=None):
        return gate_read(anchor.committed_read(q, state, dtype=torch.float32).to(q.dtype), valid, head_gate)

    @staticmethod
    def memory_commit(key, value, scores, active, chunk, state):
        anchor.commit_decode(key, value, scores, active, chunk, state)

    # ---- sampling and bookkeeping ----
    @staticmethod
    def sample(logits, attempt_ids, steps, seen, *, seed, temperature, top_k, top_p, penalty,
               backend="triton_top20"):
        """The fused top-20 sampler (inference_kernels.py:1119-1167) with the
        presence penalty."""
        sc = sampling.presence_penalty(logits, seen, penalty) if seen is not None else logits.float()
        vals, idx = torch.topk(sc / temperature, top_k, dim=-1)
        return sampling.top20_counter_sample(vals, idx, attempt_ids, steps, seed=seed, top_p=top_p)

    @staticmethod
    def bookkeeping(*args, **kw):
        slots.decode_state_update_torch(*args, **kw)


class BatchedHostOps(HostOps):
    """HostOps with the anchor memory's decode read and commit batched over
    the rows, as the reference's torch branch runs them
    (modeling_yanchor.py:283-313)."""

    @staticmethod
    def memory_read(q, state, valid=None, head_gate=None):
        return gate_read(anchor.committed_read_batched(q, state, dtype=torch.float32), valid, head_gate)

    @staticmethod
    def memory_commit(key, value, scores, active, chunk, state):
        anchor.commit_decode_batched(key, value, scores, active, chunk, state)
