"""Full-size parity of the benched path: ``MoELayer`` (bf16, the whole layer as one
autograd function) forward and backward at BASELINE.json configs C3 and C4, built
exactly as ``bench.py`` builds them (same seeds, same Zipf selection bias at C4).

* Routing is compared bit for bit with the numpy oracle (``route_topk`` from the
  logits the device computed), and so is the stable expert sort with its offsets.
* Every element of the output, the hidden states' grad, both grouped weight grads,
  the gate weight grad and the shared expert's three weight grads is compared with
  the oracle's float64 restatement run on the device (``oracle/torch_layer.py``,
  pinned against the numpy oracle on the CPU), under the bf16 storage model of the
  path (``store="bf16"``, routing weights applied to the activations: the layer
  function's ``gate_scale_on="A"``), at the north star's fixed bf16 tolerance
  |got - ref| <= 2e-2 + 2e-2 |ref|; the weight grads (sums over stored bf16 summands)
  with the summand allowance 2^-7 rss of ``helpers.TOL``.
* 48 sampled tokens (C3) / 6 (C4) are also checked end to end against the numpy
  oracle itself: out and dx are per-token functions of the token's own row.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from helpers import TOL, assert_close, close_dev, gen, np64

pytestmark = pytest.mark.gpu

RTOL = TOL[torch.bfloat16]["rtol"]
ATOL = TOL[torch.bfloat16]["atol"]


def check(got, ref, what, rss=None):
    close_dev(got, ref, what, rtol=RTOL, atol=ATOL, rss=rss)


def run_benched_layer(workload, dev):
    import bench

    T, d, E, k, f, fs, backward = bench.WORKLOADS[workload]
    assert backward
    layer = bench.build_layer(T, d, E, k, f, fs, dev)
    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    x = torch.randn(1, T, d, device=dev, generator=g).to(torch.bfloat16).requires_grad_(True)
    dout = torch.randn(1, T, d, device=dev, generator=g).to(torch.bfloat16)
    if workload == "c4":
        with torch.no_grad():
            logits = F.linear(x.detach().view(T, d), layer.gate.weight)
        bias, _, _ = bench.zipf_bias(logits, k)
        layer.gate.expert_biases.data = bias
    assert layer._fused_weights(x) is not None, "the benched whole-layer path must run"
    out, idx = layer(x)
    out.backward(dout)
    torch.cuda.synchronize()
    return layer, x, dout, out, idx, (T, d, E, k, f)


def check_full_size(workload, dev, n_sample):
    from oracle.torch_layer import TorchLayerRef
    from zmoe import ops

    print(f"[{workload}] running the benched layer fwd+bwd", flush=True)
    layer, x, dout, out, idx, (T, d, E, k, f) = run_benched_layer(workload, dev)
    x2 = x.detach().view(T, d)
    dout2 = dout.view(T, d)
    Wg = layer.gate.weight
    bias = layer.gate.expert_biases
    se_mod = layer.shared_experts
    shared = (se_mod.gate_proj.weight, se_mod.up_proj.weight, se_mod.down_proj.weight)

    # routing from the device's logits: bit for bit
    with torch.no_grad():
        logits = F.linear(x2, Wg)
    check(logits.float(), (x2.double() @ Wg.double().T).float(), "gate logits")
    logits_np = logits.float().cpu().numpy()
    ridx, rw, rp = O.route_topk(logits_np, bias.cpu().numpy(), k, round_probs_bf16=True)
    np.testing.assert_array_equal(idx.view(T, k).cpu().numpy(), ridx)
    didx, dw, dp = ops.route_topk(logits, bias, k, round_probs_bf16=True)
    np.testing.assert_array_equal(dw.cpu().numpy(), rw)
    np.testing.assert_array_equal(dp.cpu().numpy(), rp)
    # the stable expert sort and the offsets the layer used
    se, ss, off, inv = ops.flatten_sort_count(didx, E)
    r_se, r_ss, roff = O.flatten_sort_count(ridx, E)
    np.testing.assert_array_equal(se.cpu().numpy(), r_se)
    np.testing.assert_array_equal(ss.cpu().numpy(), r_ss)
    np.testing.assert_array_equal(off.cpu().numpy(), roff)
    np.testing.assert_array_equal(layer.routed_experts.last_expert_offsets.cpu().numpy(), roff)
    counts = np.diff(np.concatenate([[0], roff]))
    print(f"[{workload}] routing and sort bit-exact; rows per expert min {counts.min()} max {counts.max()}, "
          f"{int((counts == 0).sum())} empty", flush=True)

    # every element against the float64 restatement on the device
    ref = TorchLayerRef(Wg, layer.routed_experts.experts.weight, layer.routed_experts.output_experts.weight, k,
                        shared=shared, store="bf16", gate_scale_on="A", grad_dtype=torch.bfloat16)
    tidx = torch.from_numpy(ridx).to(dev)
    rout = ref.forward(x2, tidx, torch.from_numpy(rw).to(dev), torch.from_numpy(rp).to(dev))
    check(out.view(T, d), rout, "out")
    del rout
    rg = ref.backward(dout2, rss=True)
    del ref
    rss = rg.pop("rss")
    check(x.grad.view(T, d), rg["x"], "dx")
    # sums over stored bf16 summands: + 2^-7 rss (helpers.TOL)
    for what, got, key in (("dW1", layer.routed_experts.experts.weight.grad, "W1"),
                           ("dW2", layer.routed_experts.output_experts.weight.grad, "W2"),
                           ("d gate.weight", Wg.grad, "gate_weight"),
                           ("d shared gate_proj", se_mod.gate_proj.weight.grad, "shared_gate"),
                           ("d shared up_proj", se_mod.up_proj.weight.grad, "shared_up"),
                           ("d shared down_proj", se_mod.down_proj.weight.grad, "shared_down")):
        check(got, rg[key], what, rss=rss[key])
        del rg[key], rss[key]
    d_gates_ref, d_gates_rss = rg["d_gates"], rss["d_gates"]
    del rg, rss
    torch.cuda.empty_cache()

    # sampled tokens end to end against the numpy oracle (a compact stack of the experts
    # they select; out and dx of a token depend only on its own row)
    rows = torch.randperm(T, generator=gen(7))[:n_sample].sort().values
    r_np = rows.numpy()
    ids = np.unique(ridx[r_np])
    W1c = np64(layer.routed_experts.experts.weight[torch.from_numpy(ids).to(dev)])
    W2c = np64(layer.routed_experts.output_experts.weight[torch.from_numpy(ids).to(dev)])
    orc = O.MoELayerOracle(np64(Wg), bias.cpu().numpy(), W1c, W2c, k, shared=tuple(np64(w) for w in shared),
                           round_probs_bf16=True, store="bf16", gate_scale_on="A", expert_ids=ids)
    o_out, o_idx, _ = orc.forward(np64(x2[rows.to(dev)]), logits=logits_np[r_np])
    np.testing.assert_array_equal(o_idx, ridx[r_np])
    og = orc.backward(np64(dout2[rows.to(dev)]), rss=True)
    tol = TOL[torch.bfloat16]
    assert_close(np64(out.view(T, d)[rows.to(dev)]), o_out, **tol, what=f"{workload} sampled out")
    assert_close(np64(x.grad.view(T, d)[rows.to(dev)]), og["x"], **tol, what=f"{workload} sampled dx")
    # the two restatements agree (both float64; only the summation order differs)
    np.testing.assert_allclose(d_gates_ref[rows.to(dev)].cpu().numpy(), og["d_gates"], rtol=1e-9, atol=1e-9)
    np.testing.assert_allclose(d_gates_rss[rows.to(dev)].cpu().numpy(), og["rss"]["d_gates"], rtol=1e-9)


def test_c3_whole_layer_fwd_bwd(hip_device):
    """BASELINE config 3 (T=32768 d=2048 E=128 k=8 f=768, shared 1536), the bench's step."""
    check_full_size("c3", hip_device, 48)


def test_c4_whole_layer_fwd_bwd(hip_device):
    """BASELINE config 4 (T=8192 d=7168 E=256 k=8 f=2048, shared 2048, Zipf(1.1) selection
    bias), the bench's --workload c4 step."""
    check_full_size("c4", hip_device, 6)
