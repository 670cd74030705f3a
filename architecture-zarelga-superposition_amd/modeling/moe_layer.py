"""MoE sublayer (reference modeling/moe_layer.py:11-59) on MI355X.

Same submodules, parameters and state-dict keys as the reference:
``gate`` (MoEGate), ``shared_experts`` (ExpertMLP), ``routed_experts`` (GLUMLP).
The optional unpad around the layer (the reference uses flash-attn's
index_first_axis) is folded into the RMSNorm pass when the block's norm is passed
(``forward(..., norm=...)``), else a torch gather; the re-pad of the output
(pad_input) is folded into the routed experts' combine pass, which writes the padded
layout directly.
"""

import torch
import torch.nn as nn
import torch.nn.functional as F

from scattermoe.mlp import GLUMLP
from zmoe import functional as _zf
from zmoe import library as _zl

from .expert_layer import ExpertMLP
from .moe_gate import MoEGate


def index_first_axis(x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
    """Rows ``indices`` of ``x`` [N, ...] (flash_attn.bert_padding.index_first_axis)."""
    return x.index_select(0, indices)


def pad_input(x: torch.Tensor, indices: torch.Tensor, batch: int, seqlen: int) -> torch.Tensor:
    """Scatter rows back into a zero [batch, seqlen, ...] tensor (flash_attn pad_input)."""
    out = torch.zeros((batch * seqlen, *x.shape[1:]), dtype=x.dtype, device=x.device)
    out[indices] = x
    return out.view(batch, seqlen, *x.shape[1:])


class _FusedMoELayer(torch.autograd.Function):
    """The whole layer in one autograd function (bf16 on the device): gate projection and
    routing, shared expert, routed GLU experts, combine. The routing is computed as in the
    module composition (MoEGate, ExpertMLP and GLUMLP's fused path), with the same values.
    The routing weights are applied to the activations A instead of to the W2 outputs
    (w (A W2) = (w A) W2): the W1 epilogue writes A_s = w * silu(gate) * h and the combine
    sums unweighted rows. In the backward, the W2 input-grad GEMM (dA = dout[t] W2_e, W2_e
    the [d, f] weight of expert e) reads the output grad's rows in place, and one row pass
    (zmoe_swiglu_backward_gates) scales dA by w, runs the SwiGLU backward and forms the
    gates' grad <dout[t], Y> = <dout[t] W2_e, A> with A from H. The W2 grad is the sum of
    dout[t]^T A_s, dout's rows gathered in the weight-grad kernel. No [T*k, d] pass is left
    besides the forward combine, and Y is not kept. The backward also writes the shared
    expert's dH and the gate's d_logits side by side into one [T, 2fs + E] buffer:
    one GEMM against [W_up; W_gate; W_router] gives both of their input grads, one split-K
    weight-grad launch all three weight grads, and the k-sum pass adds that input grad to
    the routed experts' (one rounding; the composition runs two more GEMM launches and two
    adds over [T, d]).

    (x [T, d], gate weight, expert_biases, W1, W2, shared gate/up/down weights, k, E,
    pad_rows, pad_total) -> (out, topk_idx [T, k], expert_offsets [E]); out is [T, d], or
    with pad_rows (int64 [T]) the padded [pad_total, d] whose row pad_rows[t] is token t's.
    Every launch is a ``zmoe::`` custom op, so torch.compile traces through the function
    without a graph break.

    The weights and x may be fp32 (the reference's fp32 master weights and residual stream
    under bf16 autocast, main.py:595, :746): the function then computes on bf16 copies made
    once per forward (kept for its backward), writes the weight grads in fp32 straight from
    the kernels' fp32 accumulators (no bf16 grad and no cast pass) and returns x's grad as
    the k-sum pass's fp32 sum. The output is bf16 either way, as the reference's under
    autocast.
    """

    @staticmethod
    def forward(ctx, x, gate_w, expert_biases, W1, W2, Ws_gate, Ws_up, Ws_down, k: int, E: int, pad_rows=None,
                pad_total: int = 0):
        bf = torch.bfloat16
        ctx.f32_grads = W1.dtype == torch.float32
        ctx.x_dtype = x.dtype
        # bf16 compute copies of fp32 operands (one HIP pass each)
        cast = lambda t: t if t.dtype == bf else _zl.cast_bf16(t)  # noqa: E731
        x, W1, W2 = cast(x), cast(W1), cast(W2)
        # [up | gate | router] rows in one operand (cast with the concatenation)
        W3 = torch.cat([Ws_up, Ws_gate, gate_w], dim=0).to(bf)  # [2fs + E, d]; rows :2fs = [up | gate]
        Ws_down = Ws_down.to(bf)
        fs = Ws_up.shape[0]
        logits = F.linear(x, W3[2 * fs:])                                            # moe_gate.py:26
        idx, w, p = _zl.route_topk(logits, expert_biases, k, True)
        Hs = F.linear(x, W3[:2 * fs])
        As = _zl.swiglu(Hs)
        S = F.linear(As, Ws_down)                                                    # expert_layer.py:23-24
        se, ss, off, inv = _zl.flatten_sort_count(idx, E)                            # mlp.py:76-77
        w_sorted = w.reshape(-1).index_select(0, ss)
        H, A_s = _zl.glu_w1_forward(x, W1, se, ss, off, k, w_sorted)                 # A_s = w * A
        Y_s = _zl.grouped_mm(A_s, W2.permute(0, 2, 1), se, ss, 1, True, False, off,
                             "scatter2scatter")                                      # = w * Y
        out = _zl.combine(Y_s, None, k, S, pad_rows, pad_total)                      # moe_layer.py:48-56
        ctx.save_for_backward(x, W1, W2, W3, Ws_down, Hs, As, p, idx, w_sorted, se, ss, off, H, A_s, pad_rows)
        ctx.k, ctx.E, ctx.fs = k, E, fs
        ctx.mark_non_differentiable(idx, off)
        ctx.set_materialize_grads(False)  # no zero-filled grads for idx and off (two fill launches)
        return out, idx, off

    @staticmethod
    def backward(ctx, dout, d_idx, d_off):
        if dout is None:  # out took no part in the loss
            return (None,) * 12
        x, W1, W2, W3, Ws_down, Hs, As, p, idx, w_sorted, se, ss, off, H, A_s, pad_rows = ctx.saved_tensors
        k, E, fs = ctx.k, ctx.E, ctx.fs
        need = ctx.needs_input_grad
        f32 = ctx.f32_grads  # fp32 weight grads from the accumulators (fp32 master weights)
        dout = dout.to(x.dtype).contiguous()
        # the grad of the combine's inputs: dout for the shared expert's output (the addend),
        # gates * dout[t] for the routed rows, <dout[t], Y> for the gates
        dS = dout if pad_rows is None else dout.index_select(0, pad_rows)
        # routed experts: dA = dout[t] W2_e as a plain grouped GEMM on dS's rows read in
        # place, then one row pass for the SwiGLU backward of w * dA and the gates' grad (no
        # pass over Y; an epilogue that reads H inside the GEMM measured slower)
        dA = _zl.grouped_mm(dS, W2, se, ss, k, False, True, off, "glu_w2_backward_dh")
        dH, d_gates = _zl.swiglu_backward_gates(dA, H, w_sorted, ss)
        d_gates = d_gates.view(-1, k)
        dW2 = _zl.group_bwd_w_gather_dy(dS, ss, k, A_s, off, E, f32) if need[4] else None  # sum dout[t]^T (w A)
        dW1 = _zl.group_bwd_w(dH, x, off, E, ss, k, f32) if need[3] else None
        dXe = _zl.grouped_mm(dH, W1, se, ss, 1, True, False, off, "scatter2scatter")
        # shared expert, and the gate projection through the routing's analytic backward:
        # [d up | d gate | d_logits] side by side, one product for both input grads
        dAs = dS @ Ws_down
        dWs_down = _zl.dense_wgrad(dS, As, f32) if need[7] else None
        G = _zl.swiglu_route_backward(dAs, Hs, d_gates, p, idx, E)
        dx_dense = G @ W3                                   # shared expert + gate input grads
        dW3 = _zl.dense_wgrad(G, x, f32) if need[1] or need[5] or need[6] else None
        dx = _zl.sum_k(dXe, k, dx_dense, ctx.x_dtype == torch.float32)  # fp32 input: the fp32 sum
        part = (lambda a, b: None) if dW3 is None else (lambda a, b: dW3[a:b])
        return (dx, part(2 * fs, 2 * fs + E), None, dW1, dW2, part(fs, 2 * fs), part(0, fs), dWs_down,
                None, None, None, None)


class MoELayer(nn.Module):
    def __init__(self, config):
        super().__init__()
        self.config = config
        self.n_experts_per_token = config.n_experts_per_token
        self.gate = MoEGate(config)

        shared_intermediate = config.intermediate_size * config.n_shared_experts
        # As in the reference, n_shared_experts = 0 still yields a shared expert:
        # ExpertMLP treats intermediate_size=0 as "use config.intermediate_size"
        # (expert_layer.py:10), and forward always adds its output (moe_layer.py:47-53).
        self.shared_experts = ExpertMLP(config, intermediate_size=shared_intermediate)

        self.routed_experts = GLUMLP(
            input_size=config.hidden_size,
            hidden_size=config.intermediate_size,
            num_experts=config.n_routed_experts,
            top_k=config.n_experts_per_token,
            activation=nn.SiLU(),
        )
        # GLUMLP's ParallelExperts init at std 0.02; re-init at the config's 1/sqrt(d)
        # (moe_layer.py:27-36).
        self.reset_routed_expert_parameters()
        # bf16 on the device: the whole layer as one autograd function (_FusedMoELayer);
        # False runs the module composition (same forward values and weight grads)
        self.fused_layer = True

    def reset_routed_expert_parameters(self):
        std = self.config.initializer_range
        nn.init.normal_(self.routed_experts.experts.weight, mean=0.0, std=std)
        nn.init.normal_(self.routed_experts.output_experts.weight, mean=0.0, std=std)

    def _fused_weights(self, x):
        """The layer's weights for _FusedMoELayer, or None where the module composition runs.

        The function runs in bf16 on the device: with bf16 weights and input, or under bf16
        autocast with fp32 or bf16 weights and input (the reference's training mode: fp32
        master weights and residual stream, main.py:595, :746). Other cases (fp32 without
        autocast, the routed experts' unfused path) run the module composition."""
        se = self.shared_experts
        ws = (self.gate.weight, self.routed_experts.experts.weight, self.routed_experts.output_experts.weight,
              se.gate_proj.weight, se.up_proj.weight, se.down_proj.weight)
        bf, f32 = torch.bfloat16, torch.float32
        if torch.is_autocast_enabled("cuda"):
            dtypes_ok = (torch.get_autocast_dtype("cuda") == bf and x.dtype in (bf, f32)
                         and ws[0].dtype in (bf, f32) and all(w.dtype == ws[0].dtype for w in ws))
        else:
            dtypes_ok = x.dtype == bf and all(w.dtype == bf for w in ws)
        ok = (self.fused_layer and self.routed_experts.fused and dtypes_ok
              and x.dim() == 3 and x.is_cuda and all(w.is_cuda for w in ws)
              and self.gate.top_k == self.routed_experts.top_k
              and ws[4].shape[0] % 8 == 0 and ws[0].shape[0] % 8 == 0     # 16-byte rows of the dH | d_logits buffer
              and x.shape[-1] % 8 == 0 and ws[2].shape[2] % 8 == 0)      # and of the d- and f-wide operands
        return ws if ok else None

    def forward(self, hidden_states, unpad_indices=None, norm=None):
        """(out, topk_idx) as the reference's forward (moe_layer.py:38-59).

        ``norm`` (a ZeroCenteredRMSNorm, optional): the layer's input is
        ``norm(hidden_states)``, as the transformer block computes it before calling the
        layer (transformer_block.py:41-42); the normalisation and the unpad gather then
        run as one row pass (zmoe_rmsnorm_rows) instead of a norm pass and a gather."""
        bsz, seq_len, h = hidden_states.shape
        normed = None
        if norm is not None:
            # x = norm(hidden)[unpad_indices] in one pass; the layer sees already-gathered rows
            normed = _zf.rmsnorm_rows(hidden_states.reshape(bsz * seq_len, h), norm.weight, norm.eps,
                                      rows=unpad_indices)
            if unpad_indices is None:
                normed = normed.view(bsz, seq_len, h)
        ws = self._fused_weights(hidden_states if normed is None else normed.view(1, -1, h))
        if ws is not None:
            flat = hidden_states.reshape(bsz * seq_len, h)
            pad = (None, 0) if unpad_indices is None else (unpad_indices, bsz * seq_len)
            if normed is not None:
                x = normed.reshape(-1, h)
            else:
                x = flat if unpad_indices is None else index_first_axis(flat, unpad_indices)
            out, topk_idx, offsets = _FusedMoELayer.apply(x, ws[0], self.gate.expert_biases, *ws[1:],
                                                          self.gate.top_k, self.routed_experts.num_experts, *pad)
            self.routed_experts.last_expert_offsets = offsets
            if unpad_indices is None:
                return out.view(bsz, seq_len, h), topk_idx.view(bsz, seq_len, -1)
            return out.view(bsz, seq_len, h), pad_input(topk_idx, unpad_indices, bsz, seq_len)
        if normed is not None:
            x = normed if unpad_indices is None else normed.unsqueeze(0)
        elif unpad_indices is not None:
            flat = hidden_states.reshape(bsz * seq_len, h)
            x = index_first_axis(flat, unpad_indices).unsqueeze(0)
        else:
            x = hidden_states

        topk_idx, topk_weight = self.gate(x)
        shared_output = self.shared_experts(x)

        flat_topk_idx = topk_idx.reshape(-1, self.n_experts_per_token)
        flat_topk_weight = topk_weight.reshape(-1, self.n_experts_per_token)
        # out = shared_output + routed_output (moe_layer.py:48-53), the sum formed in the
        # routed experts' combine pass, which also writes the re-padded layout (:55-56)
        # directly when unpad_indices is given
        if unpad_indices is None:
            return self.routed_experts(x, flat_topk_weight, flat_topk_idx, residual=shared_output), topk_idx
        out = self.routed_experts(x, flat_topk_weight, flat_topk_idx, residual=shared_output,
                                  pad=(unpad_indices, bsz * seq_len))
        topk_idx = pad_input(topk_idx.squeeze(0), unpad_indices, bsz, seq_len)
        return out.view(bsz, seq_len, -1), topk_idx
