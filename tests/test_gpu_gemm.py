"""GPU parity of the grouped expert GEMMs (scatter2scatter, group_bwd_W and the
fused SwiGLU forward/backward epilogues) against the float64 oracle."""

import numpy as np
import pytest
import torch

import oracle as O
from helpers import TOL, assert_close, assert_close_fro, gen, np64, random_topk

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.bfloat16]

# (T, K, N, E, k, skew): small shapes use 128x128 tiles; R/E >= 256 with N >= 256 uses 256x256 (bf16)
SHAPES = [
    (300, 256, 512, 8, 2, 0.0),
    (2048, 512, 768, 8, 2, 0.0),
    (1500, 256, 256, 16, 4, 1.5),   # skewed: some experts empty
    (64, 128, 64, 32, 8, 0.0),      # few rows per expert
    (3, 64, 32, 8, 2, 0.0),         # tiny
    (1024, 256, 512, 8, 6, 0.0),    # k = 6: gathered rows divided by a non-power of two (256 tiles)
    (600, 128, 128, 12, 3, 0.5),    # k = 3 with 128 tiles
    (1200, 200, 264, 4, 2, 0.3),    # 256 tiles with K and N tails (K % 64 = 8)
    (600, 64, 256, 2, 2, 0.0),      # 256 tiles, a single K stage
    (120, 256, 80, 64, 4, 1.5),     # few rows per expert (weight streaming), skewed: experts past 32 rows
    (32, 128, 256, 32, 8, 0.0),     # weight streaming, 8 rows per expert
    (6000, 64, 128, 1000, 2, 0.5),  # E = 1000: tile decode with 16 experts per lane, the last lanes partial
]


def _routing(T, E, k, skew, hip_device, seed):
    from zmoe import ops

    idx = random_topk(T, E, k, seed=seed, skew=skew)
    se, ss, off, inv = ops.flatten_sort_count(idx.to(hip_device), E)
    return idx, se, ss, off, inv


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("T,K,N,E,k,skew", SHAPES)
@pytest.mark.parametrize("xg,yg", [(False, True), (True, False), (False, False), (True, True)])
@pytest.mark.parametrize("w_layout", ["param", "contiguous"])
def test_scatter2scatter(hip_device, dtype, T, K, N, E, k, skew, xg, yg, w_layout):
    from zmoe import ops

    idx, se, ss, off, _ = _routing(T, E, k, skew, hip_device, seed=T + K)
    g = gen(T * 7 + N)
    R = T * k
    X = torch.randn(R if xg else T, K, generator=g).to(dtype)
    Wp = (torch.randn(E, N, K, generator=g) / K ** 0.5).to(dtype)  # nn.Parameter layout [E, out, in]
    W = Wp.to(hip_device).permute(0, 2, 1) if w_layout == "param" else Wp.permute(0, 2, 1).contiguous().to(hip_device)
    Y = ops.scatter2scatter(X.to(hip_device), W, se, ss, 1 if xg else k, x_grouped=xg, y_grouped=yg,
                            expert_offsets=off)
    if xg:  # grouped input rows come straight from the sorted list (k folds into the row count)
        ref = O.scatter2scatter(np64(X), np64(Wp).transpose(0, 2, 1), se.cpu().numpy(), ss.cpu().numpy(), 1,
                                x_grouped=True, y_grouped=yg)
    else:
        ref = O.scatter2scatter(np64(X), np64(Wp).transpose(0, 2, 1), se.cpu().numpy(), ss.cpu().numpy(), k,
                                x_grouped=False, y_grouped=yg)
    assert_close(np64(Y), ref, **TOL[dtype], what=f"scatter2scatter xg={xg} yg={yg}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("w_layout", ["param", "contiguous"])
@pytest.mark.parametrize("case", ["many m-tiles, grouped A", "many n-tiles, gathered A"])
def test_scatter2scatter_banded_tile_order(hip_device, dtype, w_layout, case):
    """Experts with more than 16 m-tiles (A rows contiguous: n-tiles outer) or more than 16
    n-tiles (A rows gathered: m-tiles outer) take their inner tiles in bands of 8, odd bands
    reversed; every output tile must still be computed exactly once."""
    from zmoe import ops

    g = gen(41)
    if case.startswith("many m"):
        T, K, N, k, xg = 5300, 256, 520, 1, True
        idx = torch.zeros(T, k, dtype=torch.int64)
        idx[torch.randperm(T, generator=g)[:300]] = 1  # expert 0: 5000 rows (20 m-tiles of 256)
    else:
        T, K, N, k, xg = 700, 128, 4360, 2, False  # 18 n-tiles of 256 (35 of 128)
        idx = torch.stack([torch.zeros(T, dtype=torch.int64), torch.ones(T, dtype=torch.int64)], 1)
        idx[torch.randperm(T, generator=g)[:200]] = torch.tensor([1, 0])
    E = 2
    se, ss, off, _ = ops.flatten_sort_count(idx.to(hip_device), E)
    X = torch.randn(T * k if xg else T, K, generator=g).to(dtype)
    Wp = (torch.randn(E, N, K, generator=g) / K ** 0.5).to(dtype)
    W = Wp.to(hip_device).permute(0, 2, 1) if w_layout == "param" else Wp.permute(0, 2, 1).contiguous().to(hip_device)
    Y = ops.scatter2scatter(X.to(hip_device), W, se, ss, 1 if xg else k, x_grouped=xg, y_grouped=True,
                            expert_offsets=off)
    ref = O.scatter2scatter(np64(X), np64(Wp).transpose(0, 2, 1), se.cpu().numpy(), ss.cpu().numpy(),
                            1 if xg else k, x_grouped=xg, y_grouped=True)
    assert_close(np64(Y), ref, **TOL[dtype], what=f"scatter2scatter {case}")


# Rows per expert for the 256 x 256 rows launches (R / E >= 256): experts of 0-64 rows (an only m-tile
# of at most 64 rows), just past it (65, 128, 129), and partial last m-tiles of 5 and 64 rows
SMALL_TILE_COUNTS = np.array([0, 1, 17, 63, 64, 65, 300, 261, 576, 2000, 128, 129])


def _fixed_routing(counts, k, hip_device, seed):
    """Top-k slots that give expert e exactly counts[e] rows (sum(counts) divisible by k)."""
    from zmoe import ops

    slots = np.repeat(np.arange(len(counts)), counts)
    np.random.default_rng(seed).shuffle(slots)
    idx = torch.from_numpy(slots.reshape(-1, k)).to(hip_device)
    se, ss, off, _ = ops.flatten_sort_count(idx, len(counts))
    assert np.array_equal(np.diff(np.concatenate([[0], off.cpu().numpy()])), counts)
    return se, ss, off


@pytest.mark.parametrize("K", [200, 64, 120])
@pytest.mark.parametrize("xg,yg", [(False, True), (True, False)])
@pytest.mark.parametrize("w_layout", ["param", "contiguous"])
def test_scatter2scatter_small_tiles(hip_device, xg, yg, w_layout, K):
    """256 x 256 tiles that hold at most 64 rows (experts of 1-64 rows, last m-tiles of 5 and 64
    rows) beside full ones, with a partial n-tile (N = 264), for both weight layouts (B read row-
    or K-major) and both A forms (rows gathered or in place). K = 200: four stages, the last
    partial; 64: a single stage; 120: two, the second partial (the three-stage ring's edges)."""
    from zmoe import ops

    counts, k, N = SMALL_TILE_COUNTS, 2, 264
    E, R = len(counts), int(counts.sum())
    se, ss, off = _fixed_routing(counts, k, hip_device, seed=11)
    g = gen(R + N)
    X = torch.randn(R if xg else R // k, K, generator=g).to(torch.bfloat16)
    Wp = (torch.randn(E, N, K, generator=g) / K ** 0.5).to(torch.bfloat16)
    W = Wp.to(hip_device).permute(0, 2, 1) if w_layout == "param" else Wp.permute(0, 2, 1).contiguous().to(hip_device)
    Y = ops.scatter2scatter(X.to(hip_device), W, se, ss, 1 if xg else k, x_grouped=xg, y_grouped=yg,
                            expert_offsets=off)
    ref = O.scatter2scatter(np64(X), np64(Wp).transpose(0, 2, 1), se.cpu().numpy(), ss.cpu().numpy(),
                            1 if xg else k, x_grouped=xg, y_grouped=yg)
    assert_close(np64(Y), ref, **TOL[torch.bfloat16], what=f"scatter2scatter small tiles xg={xg} yg={yg}")


def test_glu_w1_forward_scaled_small_tiles(hip_device):
    """The W1 forward's SwiGLU epilogue (H and the row-scaled A) on 256 x 256 pair tiles that hold
    at most 64 rows beside full ones (f = 136: a partial pair tile; d = 200: a partial K stage)."""
    from zmoe import ops

    counts, k, d, f = SMALL_TILE_COUNTS, 2, 200, 136
    E, R = len(counts), int(counts.sum())
    se, ss, off = _fixed_routing(counts, k, hip_device, seed=12)
    g = gen(R + f)
    x = torch.randn(R // k, d, generator=g).to(torch.bfloat16)
    W1 = (torch.randn(E, 2 * f, d, generator=g) / d ** 0.5).to(torch.bfloat16)
    rs = (torch.rand(R, generator=g) + 0.05).to(hip_device)
    H, A = ops.glu_w1_forward(x.to(hip_device), W1.to(hip_device), se, ss, off, k, row_scale=rs)
    refH = O.scatter2scatter(np64(x), np64(W1).transpose(0, 2, 1), se.cpu().numpy(), ss.cpu().numpy(), k,
                             x_grouped=False, y_grouped=True)
    tol = TOL[torch.bfloat16]
    assert_close(np64(H), refH, **tol, what="H")
    refA = O.bf16_round((rs.double().cpu().numpy()[:, None] * O.swiglu(np64(H))).astype(np.float32))
    assert_close(np64(A), refA.astype(np.float64), **tol, what="scaled A")


def test_glu_w1_forward_banded_pair_tiles(hip_device):
    """SwiGLU W1 forward with f = 2200 (18 pair-column tiles of 128 pairs): banded n order."""
    from zmoe import ops

    T, d, f, E, k = 600, 128, 2200, 2, 2
    idx, se, ss, off, _ = _routing(T, E, k, 0.0, hip_device, seed=77)
    g = gen(78)
    x = torch.randn(T, d, generator=g).to(torch.bfloat16)
    W1 = (torch.randn(E, 2 * f, d, generator=g) / d ** 0.5).to(torch.bfloat16)
    H, A = ops.glu_w1_forward(x.to(hip_device), W1.to(hip_device), se, ss, off, k)
    refH = O.scatter2scatter(np64(x), np64(W1).transpose(0, 2, 1), se.cpu().numpy(), ss.cpu().numpy(), k,
                             x_grouped=False, y_grouped=True)
    tol = TOL[torch.bfloat16]
    assert_close(np64(H), refH, **tol, what="H")
    assert_close(np64(A), O.swiglu(np64(H)), **tol, what="A")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("T,K,N,E,k,skew", SHAPES)
@pytest.mark.parametrize("gather", [False, True])
def test_group_bwd_w(hip_device, dtype, T, K, N, E, k, skew, gather):
    from zmoe import ops

    idx, se, ss, off, _ = _routing(T, E, k, skew, hip_device, seed=T + N)
    g = gen(T * 3 + K)
    R = T * k
    DY = torch.randn(R, N, generator=g).to(dtype)
    X = torch.randn(T if gather else R, K, generator=g).to(dtype)
    DWt, _ = ops.group_bwd_w(DY.to(hip_device), X.to(hip_device), off, E,
                             x_gather=ss if gather else None, x_div=k)
    Xg = O.group(np64(X), ss.cpu().numpy(), fan_out=k) if gather else np64(X)
    ref, _ = O.group_bwd_w(np64(DY), Xg, off.cpu().numpy(), E)  # [E, K, N]
    if dtype == torch.float32:  # fp32 sums over up to ~2000 rows: the norm-wise fp32 bound
        assert_close_fro(np64(DWt), ref.transpose(0, 2, 1), what="group_bwd_w f32")
    else:
        assert_close(np64(DWt), ref.transpose(0, 2, 1), **TOL[dtype], what="group_bwd_w")
    counts = np.diff(np.concatenate([[0], off.cpu().numpy()]))
    for e in np.nonzero(counts == 0)[0]:
        assert not DWt[e].any(), f"empty expert {e} must get exact zeros"


@pytest.mark.parametrize("E", [4, 8])
@pytest.mark.parametrize("mode", ["x gather", "dy gather", "x gather f32"])
def test_group_bwd_w_banded_tile_order(hip_device, E, mode):
    """Weight grads with 17 (256-wide tiles, E = 4) or 33 (128-wide, E = 8) column tiles per
    expert and more than 64 tiles: m-tiles outer, the column index in bands of 8, odd bands
    reversed. Every [N, K] tile of every expert must still be computed exactly once."""
    from zmoe import ops

    T, k, N, K = 600, 2, 1096, 4104
    idx, se, ss, off, _ = _routing(T, E, k, 0.3, hip_device, seed=E + 50)
    g = gen(E * 9 + 1)
    dt = torch.bfloat16
    if mode == "dy gather":
        DY = torch.randn(T, N, generator=g).to(dt)
        X = torch.randn(T * k, K, generator=g).to(dt)
        DWt = ops.group_bwd_w_gather_dy(DY.to(hip_device), ss, k, X.to(hip_device), off, E)
        ref, _ = O.group_bwd_w(O.group(np64(DY), ss.cpu().numpy(), fan_out=k), np64(X), off.cpu().numpy(), E)
    else:
        DY = torch.randn(T * k, N, generator=g).to(dt)
        X = torch.randn(T, K, generator=g).to(dt)
        DWt, _ = ops.group_bwd_w(DY.to(hip_device), X.to(hip_device), off, E, x_gather=ss, x_div=k,
                                 out_dtype=torch.float32 if mode.endswith("f32") else None)
        ref, _ = O.group_bwd_w(np64(DY), O.group(np64(X), ss.cpu().numpy(), fan_out=k), off.cpu().numpy(), E)
    if mode.endswith("f32"):
        assert DWt.dtype == torch.float32
        assert_close_fro(np64(DWt), ref.transpose(0, 2, 1), what="group_bwd_w banded f32")
    else:
        assert_close(np64(DWt), ref.transpose(0, 2, 1), **TOL[dt], what=f"group_bwd_w banded {mode}")


@pytest.mark.parametrize("T,K,N,E,k,skew", SHAPES[:10])
def test_group_bwd_w_gather_dy(hip_device, T, K, N, E, k, skew):
    """bf16 weight grads with the gather on DY's rows: sorted row i of DY is
    DY[ss[i] // k] (the output grad's rows read in place), X in sorted order."""
    from zmoe import ops

    idx, se, ss, off, _ = _routing(T, E, k, skew, hip_device, seed=T + 5 * N)
    g = gen(T * 5 + K)
    dt = torch.bfloat16
    DY = torch.randn(T, N, generator=g).to(dt)
    X = torch.randn(T * k, K, generator=g).to(dt)
    DWt = ops.group_bwd_w_gather_dy(DY.to(hip_device), ss, k, X.to(hip_device), off, E)
    ref, _ = O.group_bwd_w(O.group(np64(DY), ss.cpu().numpy(), fan_out=k), np64(X), off.cpu().numpy(), E)
    assert_close(np64(DWt), ref.transpose(0, 2, 1), **TOL[dt], what="group_bwd_w_gather_dy")
    counts = np.diff(np.concatenate([[0], off.cpu().numpy()]))
    for e in np.nonzero(counts == 0)[0]:
        assert not DWt[e].any(), f"empty expert {e} must get exact zeros"


@pytest.mark.parametrize("k", [2, 3, 6])
def test_group_bwd_w_gather_dy_small_expert_split(hip_device, k):
    """The DY gather on both sides of the few-rows split and its k-step bounds (0, 1, 5, 16,
    17, 63, 64, 65 rows); k = 3 and 6 divide the gathered slot ids by a non-power of two."""
    from zmoe import ops

    counts = np.array([0, 1, 64, 65, 700, 2000, 300, 1000, 63, 0, 16, 17, 5])
    E, N, K = len(counts), 256, 320
    off = torch.from_numpy(np.cumsum(counts)).to(hip_device)
    R = int(counts.sum())
    g = gen(R + K)
    ss = torch.from_numpy(np.random.default_rng(8).permutation(R)).to(hip_device)
    DY = torch.randn(R // k + 1, N, generator=g).to(torch.bfloat16)
    X = torch.randn(R, K, generator=g).to(torch.bfloat16)
    DWt = ops.group_bwd_w_gather_dy(DY.to(hip_device), ss, k, X.to(hip_device), off, E)
    ref, _ = O.group_bwd_w(O.group(np64(DY), ss.cpu().numpy(), fan_out=k), np64(X), off.cpu().numpy(), E)
    assert_close(np64(DWt), ref.transpose(0, 2, 1), **TOL[torch.bfloat16], what="group_bwd_w_gather_dy split")
    for e in np.nonzero(counts == 0)[0]:
        assert not DWt[e].any(), f"empty expert {e} must get exact zeros"


@pytest.mark.parametrize("mode", ["x gather", "dy gather", "x gather f32"])
def test_group_bwd_w_skewed_expert_rounds(hip_device, mode):
    """Skewed routing (fewer than 1024 rows per expert on average) with at least 32 tiles per
    expert (N = 1024, K = 2048: 4 x 8 tiles of 256 x 256): one launch covers every expert,
    experts of at most 64 rows on the few-rows form, and the slabs are dealt round-robin over
    the experts. Row counts on both sides of the split and empty experts."""
    from zmoe import ops

    counts = np.array([0, 3, 64, 65, 1500, 17, 0, 700, 1, 2200, 63, 16, 5, 300, 129, 0])
    E, k, N, K = len(counts), 3, 1024, 2048
    off = torch.from_numpy(np.cumsum(counts)).to(hip_device)
    R = int(counts.sum())
    g = gen(R + 17)
    ss = torch.from_numpy(np.random.default_rng(11).permutation(R)).to(hip_device)
    if mode == "dy gather":
        DY = torch.randn(R // k + 1, N, generator=g).to(torch.bfloat16)
        X = torch.randn(R, K, generator=g).to(torch.bfloat16)
        DWt = ops.group_bwd_w_gather_dy(DY.to(hip_device), ss, k, X.to(hip_device), off, E)
        ref, _ = O.group_bwd_w(O.group(np64(DY), ss.cpu().numpy(), fan_out=k), np64(X), off.cpu().numpy(), E)
    else:
        DY = torch.randn(R, N, generator=g).to(torch.bfloat16)
        X = torch.randn(R // k + 1, K, generator=g).to(torch.bfloat16)
        od = torch.float32 if mode.endswith("f32") else None
        DWt, _ = ops.group_bwd_w(DY.to(hip_device), X.to(hip_device), off, E, x_gather=ss, x_div=k, out_dtype=od)
        ref, _ = O.group_bwd_w(np64(DY), O.group(np64(X), ss.cpu().numpy(), fan_out=k), off.cpu().numpy(), E)
    assert_close(np64(DWt), ref.transpose(0, 2, 1), **TOL[torch.bfloat16], what=f"group_bwd_w {mode}")
    for e in np.nonzero(counts == 0)[0]:
        assert not DWt[e].any(), f"empty expert {e} must get exact zeros"


@pytest.mark.parametrize("out_f32", [False, True])
def test_group_bwd_w_empty_experts_on_the_k_loop_launch(hip_device, out_f32):
    """At least 1024 rows per expert on average (no few-rows split): the empty experts' tiles of
    the K-loop launch write their zeros directly; every other expert's grad is unchanged."""
    from zmoe import ops

    counts = np.array([0, 3000, 5000, 0, 2100, 1])
    E, k, N, K = len(counts), 2, 512, 768
    off = torch.from_numpy(np.cumsum(counts)).to(hip_device)
    R = int(counts.sum())
    assert R >= 1024 * E
    g = gen(R + 3)
    ss = torch.from_numpy(np.random.default_rng(5).permutation(R)).to(hip_device)
    DY = torch.randn(R, N, generator=g).to(torch.bfloat16)
    X = torch.randn(R // k + 1, K, generator=g).to(torch.bfloat16)
    DWt = torch.full((E, N, K), float("nan"), dtype=torch.float32 if out_f32 else torch.bfloat16,
                     device=hip_device)  # the zeros must be written, not left from the buffer
    ops.group_bwd_w(DY.to(hip_device), X.to(hip_device), off, E, x_gather=ss, x_div=k, out=DWt,
                    out_dtype=torch.float32 if out_f32 else None)
    ref, _ = O.group_bwd_w(np64(DY), O.group(np64(X), ss.cpu().numpy(), fan_out=k), off.cpu().numpy(), E)
    if out_f32:
        assert_close_fro(np64(DWt), ref.transpose(0, 2, 1), what="group_bwd_w f32")
    else:
        assert_close(np64(DWt), ref.transpose(0, 2, 1), **TOL[torch.bfloat16], what="group_bwd_w")
    for e in np.nonzero(counts == 0)[0]:
        assert (DWt[e] == 0).all(), f"empty expert {e} must get exact zeros"


@pytest.mark.parametrize("out_f32", [False, True])
@pytest.mark.parametrize("gather", [False, True, "dy"])
def test_group_bwd_w_zero_fillers(hip_device, out_f32, gather):
    """Fewer than 1024 rows per expert on average: the empty experts' grads come from the
    zero-filler workgroups of the 256 x 256 launch with the few-rows form inline (each a
    contiguous share of their concatenation, shares crossing expert boundaries), not from their
    tiles; with the gather on DY, from the separate few-rows launch. The output starts as NaN so
    that every zero must be written. Empty experts first, last and adjacent."""
    from zmoe import ops

    if gather == "dy":
        counts = np.array([0, 0, 1, 64, 65, 700, 0, 2400, 3, 0, 0, 300, 0])
        E, k, N, K = len(counts), 2, 264, 512
        off = torch.from_numpy(np.cumsum(counts)).to(hip_device)
        R = int(counts.sum())
        g = gen(R + 6)
        ss = torch.from_numpy(np.random.default_rng(10).permutation(R)).to(hip_device)
        DY = torch.randn(R // k + 1, N, generator=g).to(torch.bfloat16)
        X = torch.randn(R, K, generator=g).to(torch.bfloat16)
        DWt = torch.full((E, N, K), float("nan"), dtype=torch.float32 if out_f32 else torch.bfloat16,
                         device=hip_device)
        ops.group_bwd_w_gather_dy(DY.to(hip_device), ss, k, X.to(hip_device), off, E, out=DWt,
                                  out_dtype=torch.float32 if out_f32 else None)
        ref, _ = O.group_bwd_w(O.group(np64(DY), ss.cpu().numpy(), fan_out=k), np64(X), off.cpu().numpy(), E)
        if out_f32:
            assert_close_fro(np64(DWt), ref.transpose(0, 2, 1), what="group_bwd_w_gather_dy f32")
        else:
            assert_close(np64(DWt), ref.transpose(0, 2, 1), **TOL[torch.bfloat16], what="group_bwd_w_gather_dy")
        for e in np.nonzero(counts == 0)[0]:
            assert (DWt[e] == 0).all(), f"empty expert {e} must get exact zeros"
        return

    counts = np.array([0, 0, 1, 64, 65, 700, 0, 2400, 3, 0, 0, 300, 0])
    E, k, N, K = len(counts), 2, 512, 264
    off = torch.from_numpy(np.cumsum(counts)).to(hip_device)
    R = int(counts.sum())
    assert 256 * E <= R < 1024 * E  # 256 x 256 tiles, few-rows form inline
    g = gen(R + 5)
    DY = torch.randn(R, N, generator=g).to(torch.bfloat16)
    if gather:
        ss = torch.from_numpy(np.random.default_rng(9).permutation(R)).to(hip_device)
        X = torch.randn(R // k + 1, K, generator=g).to(torch.bfloat16)
        Xg = O.group(np64(X), ss.cpu().numpy(), fan_out=k)
    else:
        ss = None
        X = torch.randn(R, K, generator=g).to(torch.bfloat16)
        Xg = np64(X)
    DWt = torch.full((E, N, K), float("nan"), dtype=torch.float32 if out_f32 else torch.bfloat16,
                     device=hip_device)
    ops.group_bwd_w(DY.to(hip_device), X.to(hip_device), off, E, x_gather=ss, x_div=k, out=DWt,
                    out_dtype=torch.float32 if out_f32 else None)
    ref, _ = O.group_bwd_w(np64(DY), Xg, off.cpu().numpy(), E)
    if out_f32:
        assert_close_fro(np64(DWt), ref.transpose(0, 2, 1), what="group_bwd_w f32")
    else:
        assert_close(np64(DWt), ref.transpose(0, 2, 1), **TOL[torch.bfloat16], what="group_bwd_w")
    for e in np.nonzero(counts == 0)[0]:
        assert (DWt[e] == 0).all(), f"empty expert {e} must get exact zeros"


@pytest.mark.parametrize("T,d,f,E,k,skew", [(300, 256, 512, 8, 2, 0.0), (2048, 512, 768, 8, 2, 0.0),
                                            (1200, 200, 136, 4, 2, 0.3), (128, 512, 136, 64, 4, 1.5),
                                            (32, 256, 256, 32, 8, 0.0)])
def test_glu_w1_forward_scaled(hip_device, T, d, f, E, k, skew):
    """A = row_scale * silu(gate) * h from the W1 epilogue (tiled and weight-streaming paths),
    H unchanged."""
    from zmoe import ops

    idx, se, ss, off, _ = _routing(T, E, k, skew, hip_device, seed=T + 7 * f)
    g = gen(T + 3 * d + f)
    x = torch.randn(T, d, generator=g).to(torch.bfloat16).to(hip_device)
    W1 = (torch.randn(E, 2 * f, d, generator=g) / d ** 0.5).to(torch.bfloat16).to(hip_device)
    rs = (torch.rand(T * k, generator=g) + 0.05).to(hip_device)
    H0, A0 = ops.glu_w1_forward(x, W1, se, ss, off, k)
    H, A = ops.glu_w1_forward(x, W1, se, ss, off, k, row_scale=rs)
    assert torch.equal(H, H0)
    ref = O.bf16_round((rs.double().cpu().numpy()[:, None] * O.swiglu(np64(H))).astype(np.float32))
    assert_close(np64(A), ref.astype(np.float64), **TOL[torch.bfloat16], what="scaled A")


@pytest.mark.parametrize("gather,k", [(False, 2), (True, 2), (True, 3), (True, 6)])
def test_group_bwd_w_small_expert_split(hip_device, gather, k):
    """bf16 weight grads with 256 x 256 tiles and fewer than 1024 rows per expert on average:
    experts of at most 64 rows go to the write-bound few-rows kernel (one to four 16-deep
    k-steps). Row counts at each k-step bound and on both sides of the split (0, 1, 5, 16,
    17, 63, 64, 65) beside large experts; K = 320 leaves a partial 256-column tile. With the
    x gather, k = 3 and 6 divide the slot ids by a non-power of two."""
    from zmoe import ops

    counts = np.array([0, 1, 64, 65, 700, 2000, 300, 1000, 63, 0, 16, 17, 5])
    E, N, K = len(counts), 256, 320
    off = torch.from_numpy(np.cumsum(counts)).to(hip_device)
    R = int(counts.sum())
    g = gen(R + N)
    DY = torch.randn(R, N, generator=g).to(torch.bfloat16)
    if gather:  # x rows of R / k tokens, each sorted row r reads token ss[r] // k
        ss = torch.from_numpy(np.random.default_rng(7).permutation(R)).to(hip_device)
        X = torch.randn(R // k + 1, K, generator=g).to(torch.bfloat16)
        Xg = O.group(np64(X), ss.cpu().numpy(), fan_out=k)
    else:
        ss = None
        X = torch.randn(R, K, generator=g).to(torch.bfloat16)
        Xg = np64(X)
    DWt, _ = ops.group_bwd_w(DY.to(hip_device), X.to(hip_device), off, E, x_gather=ss, x_div=k)
    ref, _ = O.group_bwd_w(np64(DY), Xg, off.cpu().numpy(), E)
    assert_close(np64(DWt), ref.transpose(0, 2, 1), **TOL[torch.bfloat16], what="group_bwd_w split")
    for e in np.nonzero(counts == 0)[0]:
        assert not DWt[e].any(), f"empty expert {e} must get exact zeros"


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("T,d,f,E,k,skew", [(300, 256, 512, 8, 2, 0.0), (2048, 512, 768, 8, 2, 0.0),
                                            (1500, 256, 96, 16, 4, 1.5), (2, 64, 32, 8, 2, 0.0),
                                            (1200, 200, 136, 4, 2, 0.3), (128, 512, 136, 64, 4, 1.5)])
def test_glu_fused_forward_and_backward_dh(hip_device, dtype, T, d, f, E, k, skew):
    from zmoe import ops

    idx, se, ss, off, _ = _routing(T, E, k, skew, hip_device, seed=T + f)
    g = gen(T + d + f)
    x = torch.randn(T, d, generator=g).to(dtype)
    W1 = (torch.randn(E, 2 * f, d, generator=g) / d ** 0.5).to(dtype)
    W2 = (torch.randn(E, d, f, generator=g) / f ** 0.5).to(dtype)
    H, A = ops.glu_w1_forward(x.to(hip_device), W1.to(hip_device), se, ss, off, k)
    refH = O.scatter2scatter(np64(x), np64(W1).transpose(0, 2, 1), se.cpu().numpy(), ss.cpu().numpy(), k,
                             x_grouped=False, y_grouped=True)
    tol = TOL[dtype]
    assert_close(np64(H), refH, **tol, what="H")
    # A is computed from the stored (rounded) H, as the reference stores H first
    assert_close(np64(A), O.swiglu(np64(H)), **tol, what="A")

    dYg = torch.randn(T * k, d, generator=g).to(dtype)
    dH = ops.glu_w2_backward_dh(dYg.to(hip_device), W2.to(hip_device), H, se, off)
    dA = O.scatter2scatter(np64(dYg), np64(W2), se.cpu().numpy(), ss.cpu().numpy(), 1, x_grouped=True,
                           y_grouped=True)
    if dtype == torch.bfloat16:
        dA = O.bf16_round(dA.astype(np.float32)).astype(np.float64)  # dA is stored in bf16 before the epilogue
    assert_close(np64(dH), O.swiglu_backward(dA, np64(H)), **tol, what="dH")


@pytest.mark.parametrize("T,d,f,E,k,skew", [(300, 256, 512, 8, 2, 0.0), (2048, 512, 768, 8, 2, 0.0),
                                            (1500, 256, 96, 16, 4, 1.5), (2, 64, 32, 8, 2, 0.0),
                                            (1200, 200, 136, 4, 2, 0.3), (128, 512, 136, 64, 4, 1.5)])
def test_glu_w2_backward_dh_gates(hip_device, T, d, f, E, k, skew):
    """The dA GEMM with the combine's backward folded in (bf16): dH from dA = gates[s] *
    (dout[s // k] @ W2[e]) and d_gates[s] = <dout[s // k], Y[s]>, Y = A W2^T, against the
    float64 oracle on the device's H and A."""
    from zmoe import ops

    idx, se, ss, off, _ = _routing(T, E, k, skew, hip_device, seed=T + 3 * f)
    g = gen(T + 2 * d + f)
    dt = torch.bfloat16
    x = torch.randn(T, d, generator=g).to(dt)
    W1 = (torch.randn(E, 2 * f, d, generator=g) / d ** 0.5).to(dt)
    W2 = (torch.randn(E, d, f, generator=g) / f ** 0.5).to(dt)
    dout = torch.randn(T, d, generator=g).to(dt)
    gates = torch.rand(T, k, generator=g) + 0.05
    H, A = ops.glu_w1_forward(x.to(hip_device), W1.to(hip_device), se, ss, off, k)
    dH, d_gates = ops.glu_w2_backward_dh_gates(dout.to(hip_device), W2.to(hip_device), H, se, ss, off, k,
                                               gates.to(hip_device))
    se_n, ss_n = se.cpu().numpy(), ss.cpu().numpy()
    dYg = O.group(np64(dout), ss_n, coeff=gates.numpy().astype(np.float64), fan_out=k)
    dA = O.scatter2scatter(dYg, np64(W2), se_n, ss_n, 1, x_grouped=True, y_grouped=True)
    dA = O.bf16_round(dA.astype(np.float32)).astype(np.float64)  # dA is stored in bf16 before the epilogue
    tol = TOL[dt]
    assert_close(np64(dH), O.swiglu_backward(dA, np64(H)), **tol, what="dH")
    Y = O.scatter2scatter(np64(A), np64(W2).transpose(0, 2, 1), se_n, ss_n, 1, x_grouped=True, y_grouped=False)
    ref = O.rowwise_sum_product(Y.reshape(T, k, d), np64(dout))
    # the kernel forms <dout[t], Y> as sum_c (dout[t] W2_e)_c A_c from its staged bf16 dA:
    # bound by the root-sum-square of those f summands (see helpers.TOL)
    dAu = O.scatter2scatter(O.group(np64(dout), ss_n, fan_out=k), np64(W2), se_n, ss_n, 1, x_grouped=True,
                            y_grouped=True)
    rss = np.empty(T * k)
    rss[ss_n] = np.sqrt(((dAu * np64(A)) ** 2).sum(axis=1))
    assert_close(d_gates.cpu().numpy().astype(np.float64), ref, **tol, what="d_gates", rss=rss.reshape(T, k))


@pytest.mark.parametrize("M,N,K,splits", [(1000, 128, 256, None), (1000, 128, 256, 3), (4100, 256, 512, 7),
                                          (4096, 136, 264, 1), (0, 128, 128, 4), (20000, 1536, 512, None),
                                          # 33..64 splits, more tiles than the GPU has CUs
                                          (40000, 512, 768, 48), (70000, 512, 768, 64), (65536, 8, 256, None)])
def test_dense_wgrad_bf16(hip_device, M, N, K, splits):
    """DW = DY^T X with split-K fp32 partials (the nn.Linear weight grads of the shared
    expert and gate projection) against float64."""
    from zmoe import ops

    g = gen(M + N + K)
    DY = torch.randn(M, N, generator=g).to(torch.bfloat16)
    X = torch.randn(M, K, generator=g).to(torch.bfloat16)
    DW = ops.dense_wgrad(DY.to(hip_device), X.to(hip_device), splits=splits)
    ref = np64(DY).T @ np64(X)
    assert_close(np64(DW), ref, **TOL[torch.bfloat16], what=f"dense_wgrad M={M} splits={splits}")


def test_dense_wgrad_f32(hip_device):
    from zmoe import ops

    g = gen(5)
    DY = torch.randn(777, 64, generator=g)
    X = torch.randn(777, 96, generator=g)
    DW = ops.dense_wgrad(DY.to(hip_device), X.to(hip_device), splits=4)
    assert_close_fro(np64(DW), np64(DY).T @ np64(X), what="dense_wgrad f32")  # 777-row fp32 sums
