"""GPU parity of the S8 polar map (every arithmetic mode) against the oracle.

Gates (north star): per-matrix relative Frobenius error vs the eager FP32
restatement <= 1e-4 in FP32-MFMA mode and <= 1e-2 in compensated-BF16 mode
(and in the mixed mode: compensated stages 1-2, FP16 stages 3-5 of an
X-space matrix, a Gram-space one compensated throughout).
The FP64 SVD closed form U f(S) V^T is checked alongside.
"""
import pytest
import torch

from oracle import sandmuon_oracle as O
from sandmuon_amd import _native
from sandmuon_amd.optimizer import _s8_fp32
from sandmuon_amd.workloads import s8_cfg2_batch

pytestmark = pytest.mark.gpu

TOL = {"fp32": 1e-4, "comp_bf16": 1e-2, "mixed": 1e-2}


def per_matrix_rel(a, b):
    a = a.double().cpu()
    b = b.double().cpu()
    return ((a - b).flatten(-2).norm(dim=-1) / b.flatten(-2).norm(dim=-1)).tolist()


@pytest.mark.parametrize("mode", ["fp32", "comp_bf16", "mixed"])
@pytest.mark.parametrize("shape", [(2, 7, 3), (2, 3, 7), (2, 4, 4), (3, 64, 96), (2, 300, 200), (1, 257, 513)])
def test_s8_small_shapes(device, mode, shape):
    torch.manual_seed(sum(shape))
    x = torch.randn(*shape)
    out = _s8_fp32(x.to(device), mode=mode)
    assert out.shape == x.shape and torch.isfinite(out).all()
    ref = O.s8(x)
    assert max(per_matrix_rel(out, ref)) <= TOL[mode]
    svd = O.s8_svd(x)
    assert max(per_matrix_rel(out, svd)) <= TOL[mode]


@pytest.mark.parametrize("mode", ["fp32", "comp_bf16", "mixed"])
@pytest.mark.parametrize("shape", [(2, 768, 768), (1, 768, 3072), (1, 3072, 768)])
def test_s8_cfg2_inputs(device, mode, shape):
    x = s8_cfg2_batch(1002 + shape[1] + shape[2], *shape)
    out = _s8_fp32(x.to(device), mode=mode)
    ref = O.s8(x)
    errs = per_matrix_rel(out, ref)
    print(mode, shape, "rel err vs fp32 oracle", errs)
    assert max(errs) <= TOL[mode]


def steep_batch(batch, rows, cols, p, seed):
    """Matrices whose singular values decay as i^-p (the shape of a low-rank
    training gradient) with random singular vectors."""
    g = torch.Generator().manual_seed(seed)
    n = min(rows, cols)
    out = []
    for _ in range(batch):
        u, _ = torch.linalg.qr(torch.randn(rows, n, generator=g, dtype=torch.float64))
        v, _ = torch.linalg.qr(torch.randn(cols, n, generator=g, dtype=torch.float64))
        out.append((u * torch.arange(1, n + 1, dtype=torch.float64) ** -p) @ v.T)
    return torch.stack(out).float()


# Error budgets on steep spectra (measured on MI355X: comp_bf16 up to 6e-4,
# mixed up to 3.4e-3, at p = 2 on the X-space and Gram-space shapes)
STEEP_TOL = {"fp32": 1e-4, "comp_bf16": 2e-3, "mixed": 5e-3}


@pytest.mark.parametrize("mode", ["fp32", "comp_bf16", "mixed"])
@pytest.mark.parametrize("p", [1.5, 2.0])
@pytest.mark.parametrize("shape", [(2, 384, 384), (2, 384, 1536), (1, 1536, 384)])
def test_s8_steep_spectra(device, mode, p, shape):
    # The case that sets the mixed mode's recipe: with steeply decaying
    # singular values, rounding of the iterate lands in the small singular
    # directions that the later stages amplify.  X-space (384 x 384) and
    # Gram space (384 x 1536, and transposed), against the FP32 oracle.
    x = steep_batch(*shape, p, 31 + shape[2])
    out = _s8_fp32(x.to(device), mode=mode)
    errs = per_matrix_rel(out, O.s8(x))
    print(f"steep p={p} {shape} {mode}: rel err vs fp32 oracle {max(errs):.3e}")
    assert max(errs) <= STEEP_TOL[mode], errs


@pytest.mark.parametrize("cols", [24, 300])  # 40 x 24: X-space; 40 x 300: Gram space
def test_s8_zero_matrix_is_zero_and_batch_neighbours_unaffected(device, cols):
    torch.manual_seed(3)
    x = torch.randn(3, 40, cols)
    x[1] = 0
    out = _s8_fp32(x.to(device))
    assert torch.equal(out[1].cpu(), torch.zeros(40, cols))
    ref = O.s8(x[[0, 2]])
    assert max(per_matrix_rel(out[[0, 2]], ref)) <= 1e-4
    zero = _s8_fp32(torch.zeros(1, 4, 3, device=device))
    assert torch.equal(zero.cpu(), torch.zeros(1, 4, 3))


def test_s8_orientation_transpose_equivariance(device):
    torch.manual_seed(5)
    x = torch.randn(2, 48, 80, device=device)
    a = _s8_fp32(x)
    b = _s8_fp32(x.transpose(-2, -1).contiguous())
    assert max(per_matrix_rel(b.transpose(-2, -1), a)) <= 1e-5


def _timed_s8(x, mode):
    from sandmuon_amd import _native
    _native.s8_timing(True)
    try:
        out = _s8_fp32(x, mode=mode)
    finally:
        _native.s8_timing(False)
    rec = _native.s8_timing_read()
    assert all(ms > 0 for ms, _, _ in rec)
    run, rec = rec[0], rec[1:]
    assert run[1] == "run" and run[2] == sum(f for _, _, f in rec)
    assert run[0] >= max(ms for ms, _, _ in rec)
    return out, [p for _, p, _ in rec], [f for _, _, f in rec]


def prod(mode, stage, gs=False):
    """MFMA FLOPs per logical FLOP of a product: 3 for the compensated
    products (every stage of comp_bf16; in mixed, stages 1 and 2, and every
    stage of a Gram-space class), 1 for FP32 and FP16 products."""
    return 3 if mode == "comp_bf16" or (mode == "mixed" and (stage <= 2 or gs)) else 1


def one_hot_flops(mode, stage, tiles, tm, waves, gs=False):
    """The square's one-hot (b/c) G MFMAs (32 x 32 x 16 each) per launch
    matrix: per tile and wave, over its 2 column tiles, 2 tm/64 K stages of
    3 (compensated) or 1 (FP32) products, or tm/64 FP16 stages of 4 (the
    scalar's hi and lo against both 16-deep halves)."""
    per = {"comp_bf16": 2 * (tm // 64) * 3, "fp32": 2 * (tm // 64)}.get(mode, (tm // 64) * 4)
    if mode == "mixed" and (stage <= 2 or gs):
        per = 2 * (tm // 64) * 3
    return tiles * waves * per * 2 * 2 * 32 * 32 * 16


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["fp32", "comp_bf16", "mixed"])
def test_s8_launch_timing_records_every_phase_x_space(device, mode):
    # oriented 300 x 500 padded to 512 x 512 (cp == rp): the stages run on
    # the iterate.  The apply computes 2 x 4 tiles of 256 x 128, the Gram
    # and the square the 10 upper-triangle 128 x 128 tiles of their 512 x 512
    # results (three matrices take fewer rounds of the CUs' block slots in
    # the smaller geometry); the square of stages 2-5 adds the one-hot MFMAs.
    x = torch.randn(3, 300, 500, device=device)
    _, phases, fl = _timed_s8(x, mode)
    assert phases == ["gram", "square", "poly1", "apply"] + ["gram", "square", "apply"] * 4
    want = []
    for stage in range(1, 6):
        f = prod(mode, stage)
        gram, apply = 3 * 10 * 2 * 128 * 128 * 512 * f, 3 * 8 * 2 * 256 * 128 * 512 * f
        square = 3 * 10 * 2 * 128 * 128 * 512 * f + (0 if stage == 1 else 3 * one_hot_flops(mode, stage, 10, 128, 4))
        want += [gram, square, 0.0, apply] if stage == 1 else [gram, square, apply]
    assert fl == want


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["fp32", "comp_bf16", "mixed"])
def test_s8_launch_timing_records_every_phase_gram_space(device, mode):
    # oriented 300 x 520 padded to 512 x 768 (cp > rp): Gram space, in two
    # segments.  Grams of X0 (stage 1) and X2 (stage 3), K = 768; applies of
    # Q2 to X0 and of Q5 to X2 over 2 x 6 tiles; symmetric r x r products
    # T = P G and G = T P (stages 1, 3, 4) and the Grams on the 10
    # upper-triangle 128 x 128 tiles (three matrices take fewer rounds of
    # the CUs' block slots in the smaller geometry) and full products
    # Q' = P Q (stages 2, 4, 5) over 2 x 4 apply tiles, all with K = 512.
    x = torch.randn(3, 300, 520, device=device)
    out, phases, fl = _timed_s8(x, mode)
    assert phases == (["gram", "square", "poly1", "sym", "sym"] + ["square", "apply", "apply"]
                      + ["gram", "square", "sym", "sym"] + ["square", "sym", "sym", "apply"]
                      + ["square", "apply", "apply"])
    gram = lambda k: 3 * 10 * 2 * 128 * 128 * 768 * prod(mode, k, gs=True)
    sym = lambda k: 3 * 10 * 2 * 128 * 128 * 512 * prod(mode, k, gs=True)
    square = lambda k: sym(k) + (0 if k == 1 else 3 * one_hot_flops(mode, k, 10, 128, 4, gs=True))
    apply_q = lambda k: 3 * 8 * 2 * 256 * 128 * 512 * prod(mode, k, gs=True)
    x_apply = lambda k: 3 * 12 * 2 * 256 * 128 * 512 * prod(mode, k, gs=True)
    assert fl == ([gram(1), square(1), 0.0, sym(1), sym(1)] + [square(2), apply_q(2), x_apply(2)]
                  + [gram(3), square(3), sym(3), sym(3)] + [square(4), sym(4), sym(4), apply_q(4)]
                  + [square(5), apply_q(5), x_apply(5)])
    ref = O.s8(x.cpu())
    assert max(per_matrix_rel(out, ref)) <= TOL[mode]


@pytest.mark.gpu
def test_s8_timing_runs_only_records_one_span_per_run(device):
    from sandmuon_amd import _native
    x = torch.randn(2, 200, 260, device=device)
    _native.s8_timing(True)
    _s8_fp32(x, mode="comp_bf16")
    _native.s8_timing(False)
    full = _native.s8_timing_read()
    _native.s8_timing(True, runs_only=True)
    try:
        _s8_fp32(x, mode="comp_bf16")
        _s8_fp32(x, mode="comp_bf16")
    finally:
        _native.s8_timing(False)
    rec = _native.s8_timing_read()
    assert [p for _, p, _ in rec] == ["run", "run"]
    assert all(ms > 0 for ms, _, _ in rec)
    assert rec[0][2] == rec[1][2] == full[0][2]


@pytest.mark.parametrize("mode", ["fp32", "comp_bf16", "mixed"])
@pytest.mark.parametrize("shape", [(2, 7, 3), (3, 64, 96), (2, 300, 200), (1, 257, 513), (4, 512, 512), (3, 300, 520),
                                   (1, 520, 300), (2, 768, 3072)])
def test_s8_256x256_tiles(device, mode, shape):
    """Every GEMM launch on 256 x 256 tiles of 8 waves (forced): X-space and
    Gram-space classes, transposed inputs, a batch split over two launch
    chains, against the oracle and the SVD closed form."""
    prev = _native.s8_tile_geometry(1)
    try:
        torch.manual_seed(sum(shape) + 7)
        x = torch.randn(*shape)
        out = _s8_fp32(x.to(device), mode=mode)
    finally:
        _native.s8_tile_geometry(prev)
    assert out.shape == x.shape and torch.isfinite(out).all()
    assert max(per_matrix_rel(out, O.s8(x))) <= TOL[mode]
    assert max(per_matrix_rel(out, O.s8_svd(x))) <= TOL[mode]


@pytest.mark.parametrize("mode", ["fp32", "comp_bf16", "mixed"])
def test_s8_launch_timing_256x256_tiles(device, mode):
    # oriented 300 x 500 padded to 512 x 512 with every launch forced to
    # 256 x 256 tiles of 8 waves: the Gram and the square compute the 3
    # upper-triangle blocks of their 512 x 512 results, the apply 2 x 2
    # tiles; the one-hot term adds, per square tile and wave, 8 K stages of
    # 2 MFMA tiles 32 x 32 x 16.
    x = torch.randn(3, 300, 500, device=device)
    prev = _native.s8_tile_geometry(1)
    try:
        out, phases, fl = _timed_s8(x, mode)
    finally:
        _native.s8_tile_geometry(prev)
    assert phases == ["gram", "square", "poly1", "apply"] + ["gram", "square", "apply"] * 4
    want = []
    for stage in range(1, 6):
        f = prod(mode, stage)
        sym, apply = 3 * 3 * 2 * 256 * 256 * 512 * f, 3 * 4 * 2 * 256 * 256 * 512 * f
        square = sym + (0 if stage == 1 else 3 * one_hot_flops(mode, stage, 3, 256, 8))
        want += [sym, square, 0.0, apply] if stage == 1 else [sym, square, apply]
    assert fl == want
    assert max(per_matrix_rel(out, O.s8(x.cpu()))) <= TOL[mode]


# (tile rows, tile columns, waves) of each geometry
GEOMETRY = {"128x128": (128, 128, 4), "256x128": (256, 128, 4), "256x256": (256, 256, 8)}


def expected_square_geometry(n, size, cus):
    """The square's geometry for a launch over n matrices of size x size:
    256 x 256 tiles when there are at least 1.5 of them per CU, else 128 x 128
    tiles when they take fewer rounds of the CUs' block slots (three per CU,
    a round counted 0.9 of one of two 256 x 128 blocks), else 256 x 128."""
    t256, ts = size // 256, size // 128
    sym = lambda t: t * (t + 1) // 2
    if 2 * n * sym(t256) >= 3 * cus:
        return "256x256", sym(t256)
    big_rounds = -(-n * 2 * sym(t256) // (2 * cus))
    small_rounds = -(-n * sym(ts) // (3 * cus))
    return ("128x128", sym(ts)) if 0.9 * small_rounds < big_rounds else ("256x128", 2 * sym(t256))


@pytest.mark.parametrize("mode", ["fp32", "comp_bf16", "mixed"])
@pytest.mark.parametrize("batch,size,geometry", [(8, 512, "128x128"), (74, 768, "256x128"), (800, 256, "256x256")])
def test_s8_square_tile_geometries(device, mode, batch, size, geometry):
    """The square phase takes 256 x 256 tiles when the launch has at least
    1.5 of them per CU, else 128 x 128 tiles when they need fewer rounds of
    the CUs' block slots, else 256 x 128 tiles.  A class of 4 or more
    matrices runs as two launch chains of halves, and each chain's launches
    decide for themselves: 4 matrices of 512 x 512 on 256 CUs give 40 small
    tiles against 24 of 256 x 128, one round each; 37 of 768 x 768 give 777
    small tiles (two rounds of three per CU) against 444 of 256 x 128 (one
    round of two) and 222 of 256 x 256; 400 of 256 x 256 give 400 tiles of
    256 x 256.  Every geometry meets the gates; the recorded square FLOPs
    show which one ran."""
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    chains = [batch - batch // 2, batch // 2] if batch >= 4 else [batch]
    for n in chains:
        assert expected_square_geometry(n, size, cus)[0] == geometry, "the case no longer selects the geometry it names"
    torch.manual_seed(batch)
    x = torch.randn(batch, size, size)
    from sandmuon_amd import _native
    _native.s8_timing(True)
    try:
        out = _s8_fp32(x.to(device), mode=mode)
    finally:
        _native.s8_timing(False)
    rec = _native.s8_timing_read()
    tm, tn, waves = GEOMETRY[geometry]
    tiles = expected_square_geometry(chains[0], size, cus)[1]
    # per matrix: stage 1 (G G) and stages 2-5 (G G plus the one-hot (b/c) G
    # MFMAs)
    fs = [tiles * 2 * tm * tn * size * prod(mode, k) + (0 if k == 1 else one_hot_flops(mode, k, tiles, tm, waves))
          for k in range(1, 6)]
    want = sorted(n * f for n in chains for f in fs)
    assert sorted(f for _, p, f in rec if p == "square") == want
    errs = per_matrix_rel(out, O.s8(x))
    assert max(errs) <= TOL[mode]
