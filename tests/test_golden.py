"""Golden fixtures (tests/golden/moe_golden.npz, written by tests/golden/make_golden.py
from the CPU oracle): the oracle must still reproduce them, and the HIP path must
match them — routing and sort bit-exactly, floats within the north-star tolerances
elementwise, |got - ref| <= atol + rtol |ref| (fp32 1e-5, bf16 2e-2). The oracle's own
reproduction of the fixtures is checked at 1e-10 (absolute part relative to max|ref|)."""

import os
import sys

import numpy as np
import pytest
import torch

from helpers import TOL, assert_close, np64

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden", "moe_golden.npz")


@pytest.fixture(scope="module")
def fx():
    with np.load(GOLDEN, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_oracle_reproduces_golden(fx):
    sys.path.insert(0, os.path.join(HERE, "golden"))
    try:
        import make_golden
    finally:
        sys.path.pop(0)
    fresh = make_golden.build()
    assert sorted(fresh) == sorted(fx)
    for k, ref in fx.items():
        got = fresh[k]
        assert got.dtype == ref.dtype and got.shape == ref.shape, k
        if np.issubdtype(ref.dtype, np.integer):
            assert np.array_equal(got, ref), k
        else:
            # same inputs, same float64 arithmetic; allow BLAS summation-order ulps
            assert np.allclose(got, ref, rtol=1e-10, atol=1e-10 * max(1.0, float(np.nanmax(np.abs(ref)))),
                               equal_nan=True), k


# ----------------------------------------------------------------------------- GPU
def _t(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    return (t if dtype is None else t.to(dtype)).to(dev)


@pytest.mark.gpu
@pytest.mark.parametrize("bf16", [False, True])
def test_golden_routing(hip_device, fx, bf16):
    from zmoe import ops

    sfx = "_bf16" if bf16 else ""
    logits = _t(fx["route_logits" + sfx], hip_device, torch.bfloat16 if bf16 else torch.float32)
    idx, w, p = ops.route_topk(logits, _t(fx["route_bias"], hip_device), int(fx["route_k"]), round_probs_bf16=bf16)
    assert np.array_equal(idx.cpu().numpy(), fx["route_idx" + sfx])
    assert_close(w.cpu().numpy(), fx["route_w" + sfx], **TOL[torch.float32], what="routing weights")
    assert_close(p.cpu().numpy(), fx["route_p" + sfx], **TOL[torch.float32], what="selected probabilities")


@pytest.mark.gpu
def test_golden_sort(hip_device, fx):
    from zmoe import ops

    se, ss, off, inv = ops.flatten_sort_count(_t(fx["sort_ids"], hip_device), int(fx["sort_E"]))
    assert np.array_equal(se.cpu().numpy(), fx["sort_se"])
    assert np.array_equal(ss.cpu().numpy(), fx["sort_ss"])
    assert np.array_equal(off.cpu().numpy(), fx["sort_off"])
    assert np.array_equal(inv.cpu().numpy().astype(np.int64), fx["sort_inv"])


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_golden_gemms(hip_device, fx, dtype):
    from zmoe import ops

    E = int(fx["gemm_E"])
    k = fx["gemm_ids"].shape[1]
    se, ss, off, _ = ops.flatten_sort_count(_t(fx["gemm_ids"], hip_device), E)
    X, Xg = _t(fx["gemm_X"], hip_device, dtype), _t(fx["gemm_Xg"], hip_device, dtype)
    W = _t(fx["gemm_W"], hip_device, dtype)                          # [E, K, N]
    tol = TOL[dtype]
    Y = ops.group(X, ss, coeff=_t(fx["gemm_coeff"], hip_device), fan_out=k)
    assert_close(np64(Y), fx["gemm_group"], **tol, what="group")
    for xg in (False, True):
        for yg in (False, True):
            Y = ops.scatter2scatter(Xg if xg else X, W, se, ss, 1 if xg else k, x_grouped=xg, y_grouped=yg,
                                    expert_offsets=off)
            assert_close(np64(Y), fx[f"gemm_s2s_{int(xg)}{int(yg)}"], **tol, what=f"scatter2scatter xg={xg} yg={yg}")
    DY = _t(fx["gemm_DY"], hip_device, dtype)
    DWt, _ = ops.group_bwd_w(DY, Xg, off, E)                          # [E, N, K]
    assert_close(np64(DWt), fx["gemm_wgrad"].transpose(0, 2, 1), **tol, what="group_bwd_w")
    DWt, _ = ops.group_bwd_w(DY, X, off, E, x_gather=ss, x_div=k)
    assert_close(np64(DWt), fx["gemm_wgrad_gather"].transpose(0, 2, 1), **tol, what="group_bwd_w (gathered x)")


@pytest.mark.gpu
def test_golden_layer(hip_device, fx):
    from modeling.model_config import ModelConfig
    from modeling.moe_layer import MoELayer

    x = fx["layer_x"]
    T, d = x.shape
    E, f2, _ = fx["layer_W1"].shape
    k = int(fx["layer_k"])
    fs = fx["layer_Ws_gate"].shape[0]
    cfg = ModelConfig(hidden_size=d, intermediate_size=f2 // 2, n_experts=E + fs // (f2 // 2),
                      n_shared_experts=fs // (f2 // 2), n_experts_per_token=k)
    layer = MoELayer(cfg)
    with torch.no_grad():
        layer.gate.weight.copy_(torch.from_numpy(fx["layer_Wg"]))
        layer.gate.expert_biases.copy_(torch.from_numpy(fx["layer_bias"]))
        layer.routed_experts.experts.weight.copy_(torch.from_numpy(fx["layer_W1"]))
        layer.routed_experts.output_experts.weight.copy_(torch.from_numpy(fx["layer_W2"]))
        layer.shared_experts.gate_proj.weight.copy_(torch.from_numpy(fx["layer_Ws_gate"]))
        layer.shared_experts.up_proj.weight.copy_(torch.from_numpy(fx["layer_Ws_up"]))
        layer.shared_experts.down_proj.weight.copy_(torch.from_numpy(fx["layer_Ws_down"]))
    layer = layer.to(hip_device)
    xt = _t(x, hip_device).view(1, T, d).requires_grad_(True)
    out, idx = layer(xt)
    out.backward(_t(fx["layer_dout"], hip_device).view(1, T, d))
    tol = TOL[torch.float32]
    assert np.array_equal(idx.view(T, k).cpu().numpy(), fx["layer_idx"])
    assert_close(np64(out.view(T, d)), fx["layer_out"], **tol, what="layer output")
    se = layer.shared_experts
    for name, got, key in (("dx", xt.grad.view(T, d), "layer_dx"), ("dW gate", layer.gate.weight.grad, "layer_dWg"),
                           ("dW1", layer.routed_experts.experts.weight.grad, "layer_dW1"),
                           ("dW2", layer.routed_experts.output_experts.weight.grad, "layer_dW2"),
                           ("dW shared gate", se.gate_proj.weight.grad, "layer_dWs_gate"),
                           ("dW shared up", se.up_proj.weight.grad, "layer_dWs_up"),
                           ("dW shared down", se.down_proj.weight.grad, "layer_dWs_down")):
        assert_close(np64(got), fx[key], **tol, what=name)
