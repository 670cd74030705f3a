"""Regression fixtures for the MoE hot path, written by the CPU oracle.

The reference ships no golden vectors, known-answer tests or fixtures for this path
(it has no tests for the MoE layer at all), and every oracle function is pinned by
the checks in ``tests/test_oracle.py`` (closed forms, brute force, autograd of an
independent formulation, finite differences), so the reference was never imported
to produce vectors. These fixtures freeze the oracle's outputs on small seeded
inputs that include the reference's edge cases (ties, NaN logits, a forcing bias,
empty experts, every gather/scatter mode): ``tests/test_golden.py`` checks that the
oracle still reproduces them (CPU) and that the HIP path matches them (GPU).

    python tests/golden/make_golden.py     # rewrites tests/golden/moe_golden.npz
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle as O  # noqa: E402

OUT = os.path.join(HERE, "moe_golden.npz")


def bf16_grid(x):
    """Round float32 values to the nearest bf16 (so bf16 and fp32 paths see the same inputs)."""
    return O.bf16_round(np.asarray(x, np.float32)).astype(np.float32)


def routing_case(rng):
    T, E, k = 48, 16, 4
    logits = rng.standard_normal((T, E)).astype(np.float32)
    logits[8] = 0.25                     # all scores equal: experts 0..k-1, in order
    logits[9, :] = np.repeat(rng.standard_normal(E // 2).astype(np.float32), 2)  # pairwise ties
    logits[10, 3] = np.nan               # NaN ranks first (torch.topk's order)
    logits[11, :] = -3.0
    bias = (0.1 * rng.standard_normal(E)).astype(np.float32)
    bias[13] = 50.0                      # forces expert 13 into every top-k; its weight keeps the unbiased p
    idx, w, p = O.route_topk(logits, bias, k)
    lb = bf16_grid(logits)
    idx_b, w_b, p_b = O.route_topk(lb, bias, k, round_probs_bf16=True)
    return dict(route_logits=logits, route_bias=bias, route_k=np.int64(k), route_idx=idx, route_w=w, route_p=p,
                route_logits_bf16=lb, route_idx_bf16=idx_b, route_w_bf16=w_b, route_p_bf16=p_b)


def sort_case(rng):
    T, k, E = 40, 3, 8
    choices = np.array([0, 1, 2, 3, 4, 6, 7])   # expert 5 gets no rows
    ids = np.stack([rng.choice(choices, size=k, replace=False) for _ in range(T)]).astype(np.int64)
    se, ss, off = O.flatten_sort_count(ids, E)
    inv = O.inverse_permutation(ss)
    return dict(sort_ids=ids, sort_E=np.int64(E), sort_se=se, sort_ss=ss, sort_off=off, sort_inv=inv)


def gemm_case(rng):
    """Grouped GEMMs on one routing: group (+coeff), scatter2scatter in its four
    gather/scatter modes, group_bwd_w with and without gathered x."""
    T, k, E, K, N = 24, 2, 4, 32, 24
    ids = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int64)
    se, ss, off = O.flatten_sort_count(ids, E)
    R = T * k
    X = bf16_grid(rng.standard_normal((T, K)))
    Xg = bf16_grid(rng.standard_normal((R, K)))
    W = bf16_grid(rng.standard_normal((E, K, N)) / np.sqrt(K))     # [E, K, N] as ops.scatter2scatter takes it
    coeff = rng.random(R).astype(np.float32)
    d = dict(gemm_ids=ids, gemm_E=np.int64(E), gemm_X=X, gemm_Xg=Xg, gemm_W=W, gemm_coeff=coeff,
             gemm_group=O.group(X, ss, coeff=coeff, fan_out=k))
    for xg in (False, True):
        for yg in (False, True):
            A = Xg if xg else X
            d[f"gemm_s2s_{int(xg)}{int(yg)}"] = O.scatter2scatter(A, W, se, ss, 1 if xg else k,
                                                                   x_grouped=xg, y_grouped=yg)
    DY = bf16_grid(rng.standard_normal((R, N)))
    d["gemm_DY"] = DY
    d["gemm_wgrad"], _ = O.group_bwd_w(DY, Xg, off, E)                          # [E, K, N]
    d["gemm_wgrad_gather"], _ = O.group_bwd_w(DY, O.group(X, ss, fan_out=k), off, E)
    return d


def layer_case(rng):
    """MoELayer forward + backward (fp32) with a shared expert; the routing margin is
    checked so that ulp-level differences in the device's gate projection cannot flip
    a selection."""
    T, d, E, k, f, fs = 32, 32, 8, 2, 16, 16
    std = 1.0 / np.sqrt(d)
    for attempt in range(100):
        x = rng.standard_normal((T, d)).astype(np.float32)
        Wg = (rng.standard_normal((E, d)) * std).astype(np.float32)
        bias = (0.1 * rng.standard_normal(E)).astype(np.float32)
        s = O.sigmoid_f32((x.astype(np.float64) @ Wg.T.astype(np.float64)).astype(np.float32)) + bias
        srt = -np.sort(-s, axis=1)
        if (srt[:, k - 1] - srt[:, k]).min() > 2e-3:
            break
    else:
        raise RuntimeError("no well-separated routing found")
    W1 = (rng.standard_normal((E, 2 * f, d)) * std).astype(np.float32)
    W2 = (rng.standard_normal((E, d, f)) * std).astype(np.float32)
    shared = tuple((rng.standard_normal(sh) * std).astype(np.float32) for sh in ((fs, d), (fs, d), (d, fs)))
    dout = rng.standard_normal((T, d)).astype(np.float32)
    orc = O.MoELayerOracle(Wg, bias, W1, W2, k, shared=shared)
    out, idx, w = orc.forward(x)
    g = orc.backward(dout)
    return dict(layer_x=x, layer_Wg=Wg, layer_bias=bias, layer_W1=W1, layer_W2=W2, layer_Ws_gate=shared[0],
                layer_Ws_up=shared[1], layer_Ws_down=shared[2], layer_dout=dout, layer_k=np.int64(k),
                layer_out=out, layer_idx=idx, layer_w=w, layer_dx=g["x"], layer_dWg=g["gate_weight"],
                layer_dW1=g["W1"], layer_dW2=g["W2"], layer_dWs_gate=g["shared_gate"], layer_dWs_up=g["shared_up"],
                layer_dWs_down=g["shared_down"])


def build() -> dict:
    O.set_precision(np.float64)
    rng = np.random.default_rng(20261202)
    fx = {}
    for case in (routing_case, sort_case, gemm_case, layer_case):
        fx.update(case(rng))
    return fx


if __name__ == "__main__":
    fx = build()
    np.savez_compressed(OUT, **fx)
    print(f"wrote {OUT}: {len(fx)} arrays, {os.path.getsize(OUT)} bytes")
