"""Pins of the CPU oracle that do not retype its formulas: dense-matrix
identities, closed forms, the SVD form of S8, a library AdamW, float64
brute force, the reference's own test intents (tests/test_optimizer.py), and
planted mistakes that each pin must catch."""
import copy
import math

import numpy as np
import pytest
import torch
from torch import nn

from oracle import sandmuon_oracle as O

# paper/main.tex:196-205 table and reproduction/paper/s8/data/completed/
# s8_manifest.json:79-108 (second source for the coefficient schedule).
MANIFEST_COEFFICIENTS = [
    [11.062126275847973, -56.051653229128085, 72.32081107619855],
    [4.100720073616268, -2.9324183165353577, 0.5339692084282731],
    [3.930310192522361, -2.873509793709714, 0.5366557527206212],
    [3.280567968245866, -2.414925589994015, 0.48635134757825227],
    [2.282741575232451, -1.6302296637355072, 0.40275720810675486],
]


def test_coefficients_match_manifest():
    assert [list(c) for c in O.S8_COEFFICIENTS] == MANIFEST_COEFFICIENTS
    assert O.S8_MARGIN == 1.35 and O.S8_MULTIPLIER == 1.0
    import sandmuon_amd.coefficients as C
    assert C.S8_COEFFICIENTS == O.S8_COEFFICIENTS and C.S8_MARGIN == O.S8_MARGIN


# ------------------------------------------------------------ factors ---
def dense_whitener(second, mean, fn=O.rank1_inverse_sqrt):
    inv, z, k = fn(second, mean)
    return (torch.eye(second.numel(), dtype=second.dtype) + k * torch.outer(z, z)) @ torch.diag(inv)


def covariance_identity(fn=O.rank1_inverse_sqrt):
    # tests/test_optimizer.py:24-33: W (A / mean(second)) W^T = I.
    torch.manual_seed(7)
    x = torch.randn(500, 6, dtype=torch.float64) + torch.randn(6, dtype=torch.float64)
    second, mean = x.square().mean(0), x.mean(0)
    w = dense_whitener(second, mean, fn)
    cov = torch.diag(second - mean.square()) + torch.outer(mean, mean)
    torch.testing.assert_close(w @ (cov / second.mean()) @ w.T, torch.eye(6, dtype=torch.float64),
                               atol=1e-10, rtol=1e-10)


def test_rank1_inverse_sqrt_whitens_dense_covariance():
    covariance_identity()


def test_planted_kappa_sign_error_is_caught():
    def wrong(second, mean):
        inv, z, k = O.rank1_inverse_sqrt(second, mean)
        return inv, z, -k
    with pytest.raises(AssertionError):
        covariance_identity(wrong)


def test_diagonal_inverse_sqrt_closed_form_and_zero_signal():
    v = torch.tensor([4.0, 1.0, 0.0, 1e-9], dtype=torch.float64)
    m = v.mean().item()  # 1.25
    expect = torch.tensor([(4 / m) ** -.5, (1 / m) ** -.5, 1e-6 ** -.5, 1e-6 ** -.5], dtype=torch.float64)
    torch.testing.assert_close(O.diagonal_inverse_sqrt(v), expect)
    assert torch.isfinite(O.diagonal_inverse_sqrt(torch.zeros(4))).all()


# --------------------------------------------------- whiten / mapback ---
def test_rank1_whiten_equals_dense_two_sided_product():
    # tests/test_optimizer.py:35-43
    torch.manual_seed(7)
    x = torch.randn(500, 6, dtype=torch.float64) + torch.randn(6, dtype=torch.float64)
    second, mean = x.square().mean(0), x.mean(0)
    left = O.rank1_inverse_sqrt(second, mean)
    right = O.rank1_inverse_sqrt(second[:4], mean[:4])
    src = torch.randn(2, 6, 4, dtype=torch.float64)
    out = O.rank1_whiten(src, tuple(t.expand(2, *t.shape) if t.ndim else t.expand(2) for t in left),
                         tuple(t.expand(2, *t.shape) if t.ndim else t.expand(2) for t in right))
    wl, wr = dense_whitener(second, mean), dense_whitener(second[:4], mean[:4])
    torch.testing.assert_close(out, torch.stack([wl @ m @ wr.T for m in src]), atol=1e-10, rtol=1e-10)


def test_rank1_mapback_equals_dense_product():
    # tests/test_optimizer.py:46-54
    torch.manual_seed(8)
    q = torch.randn(5, 3, dtype=torch.float64)
    li, lz, lc = O.rank1_inverse_sqrt(torch.rand(5, dtype=torch.float64) + .3, torch.randn(5, dtype=torch.float64) * .1)
    ri, rz, rc = O.rank1_inverse_sqrt(torch.rand(3, dtype=torch.float64) + .3, torch.randn(3, dtype=torch.float64) * .1)
    expect = (torch.diag(li) @ (torch.eye(5, dtype=q.dtype) + lc * torch.outer(lz, lz)) @ q
              @ (torch.eye(3, dtype=q.dtype) + rc * torch.outer(rz, rz)) @ torch.diag(ri))
    torch.testing.assert_close(O.rank1_mapback(q, (li, lz, lc), (ri, rz, rc)), expect)


def test_graft_norm_and_reference_zero_behaviour():
    v = torch.randn(7, 3)
    assert abs(O.graft_direction(v, 7).norm().item() - math.sqrt(7)) < 1e-5
    assert torch.equal(O.graft_direction(torch.zeros(3, 4), 3), torch.zeros(3, 4))
    # sandmuon/optimizer.py:63-66: for >= 16 rows sqrt(rows)/FLT_MIN overflows
    # and a zero direction becomes NaN (a reference edge case, not copied
    # by the GPU build).
    assert torch.isnan(O.graft_direction(torch.zeros(16, 4), 16)).all()


# ------------------------------------------------------------------ S8 ---
def test_stage_polynomial_via_numpy_polyval():
    # The scalar composition against numpy's polynomial evaluator:
    # p(t) = t (a + b t^2 + c t^4) as coefficients [c, 0, b, 0, a, 0].
    t = np.linspace(1e-4, 1 / 1.35, 50)
    ref = t.copy()
    for a, b, c in MANIFEST_COEFFICIENTS:
        ref = np.polyval([c, 0, b, 0, a, 0], ref)
    sigma = torch.from_numpy(t * 1.35)
    got = O.s8_scalar(sigma, torch.ones((), dtype=torch.float64), O.S8_COEFFICIENTS, O.S8_MARGIN).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-12)


def test_s8_diagonal_input_maps_singular_values():
    # X = diag(sigma) (padded): S8(X) = diag(f(sigma)).
    sigma = torch.tensor([3.0, 1.0, 0.5, 1e-3], dtype=torch.float64)
    x = torch.zeros(4, 6, dtype=torch.float64)
    x[range(4), range(4)] = sigma
    sensor = (sigma ** 8).sum() ** 0.125
    f = O.s8_scalar(sigma, sensor)
    expect = torch.zeros(4, 6, dtype=torch.float64)
    expect[range(4), range(4)] = f
    torch.testing.assert_close(O.s8(x), expect, atol=1e-12, rtol=1e-10)


@pytest.mark.parametrize("shape", [(2, 7, 3), (2, 3, 7), (2, 4, 4), (1, 40, 64)])
def test_s8_matches_svd_closed_form(shape):
    torch.manual_seed(13)
    x = torch.randn(*shape, dtype=torch.float64)
    torch.testing.assert_close(O.s8(x), O.s8_svd(x), atol=1e-10, rtol=1e-9)
    y32 = O.s8(x.float())
    assert ((y32.double() - O.s8_svd(x)).norm() / O.s8_svd(x).norm()) < 1e-4


def test_planted_transposed_gram_is_caught():
    # A stage built on X^T X (the wrong Gram) applied from the left: valid
    # shapes for a square input, wrong map.  The SVD closed form rejects it.
    def wrong(x):
        x = x / torch.linalg.matrix_norm(x, keepdim=True)
        g = x.transpose(-2, -1) @ x
        g2 = g @ g
        s = O.S8_MARGIN * torch.linalg.matrix_norm(g2, keepdim=True) ** .25
        eye = torch.eye(x.shape[-1], dtype=x.dtype)
        a, b, c = O.S8_COEFFICIENTS[0]
        x = ((a * eye + b * g / s ** 2 + c * g2 / s ** 4) @ x) / s
        for a, b, c in O.S8_COEFFICIENTS[1:]:
            g = x.transpose(-2, -1) @ x
            x = (a * eye + b * g + c * g @ g) @ x
        return x
    torch.manual_seed(2)
    x = torch.randn(1, 6, 6, dtype=torch.float64)
    assert not torch.allclose(wrong(x), O.s8_svd(x), atol=1e-3)
    torch.testing.assert_close(O.s8(x), O.s8_svd(x), atol=1e-10, rtol=1e-9)


def test_planted_missing_schatten_scale_is_caught():
    def no_scale(x):
        saved = O.S8_MARGIN
        try:
            return O.s8(x, margin=1.0 / 1e6)  # margin slip: wrong sensor scaling
        finally:
            assert saved == O.S8_MARGIN
    x = torch.randn(1, 6, 9, dtype=torch.float64)
    assert not torch.allclose(no_scale(x), O.s8_svd(x), atol=1e-6)


def test_s8_orientation_and_zero():
    # tests/test_optimizer.py:140-149
    torch.manual_seed(13)
    for shape in ((7, 3), (3, 7), (4, 4)):
        x = torch.randn(2, *shape)
        y = O.s8(x)
        assert y.shape == x.shape and torch.isfinite(y).all()
        torch.testing.assert_close(O.s8(x.transpose(-2, -1)).transpose(-2, -1), y)
    assert torch.equal(O.s8(torch.zeros(1, 4, 3)), torch.zeros(1, 4, 3))


# --------------------------------------------------------------- stats ---
def test_accumulate_rows_float64_brute_force():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(4, 37, 19, generator=g) * 3 + 1
    sq, fs = torch.zeros(19), torch.zeros(19)
    n = O.accumulate_rows(x, sq, fs)
    assert n == 4 * 37
    flat = x.reshape(-1, 19).double()
    torch.testing.assert_close(sq.double(), (flat ** 2).sum(0), rtol=1e-6, atol=0)
    torch.testing.assert_close(fs.double(), flat.sum(0), rtol=1e-5, atol=1e-5)


def test_nesterov_closed_form():
    m, g = torch.randn(5, 3), torch.randn(5, 3)
    m0 = m.clone()
    src = O.nesterov(m, g, .8)
    torch.testing.assert_close(m, .8 * m0 + .2 * g)
    torch.testing.assert_close(src, .8 * (.8 * m0 + .2 * g) + .2 * g)


def test_adamw_matches_torch_optim_adamw():
    torch.manual_seed(4)
    p1 = torch.randn(50, requires_grad=False)
    p2 = nn.Parameter(p1.clone())
    ref = torch.optim.AdamW([p2], lr=1e-3, betas=(.9, .999), eps=1e-8, weight_decay=.01)
    st = {}
    for _ in range(3):
        g = torch.randn(50)
        O.adamw(p1, g, st, 1e-3)
        p2.grad = g.clone()
        ref.step()
        torch.testing.assert_close(p1, p2.detach(), rtol=1e-6, atol=1e-7)
    assert st["step"] == 3 and isinstance(st["step"], int)


class Proj(nn.Module):
    def __init__(self, rows, cols):
        super().__init__()
        self.proj = nn.Linear(cols, rows, bias=False)

    def forward(self, x):
        return self.proj(x)


def test_statistics_over_uneven_microbatches_analytic():
    # tests/test_optimizer.py:57-85
    torch.manual_seed(10)
    model = Proj(3, 4)
    x, target = torch.randn(9, 4), torch.randn(9, 3)
    pred0 = model(x).detach()
    expect_b = (2 * (pred0 - target) / 9).square().mean(0)
    expect_b = expect_b / expect_b.mean()
    opt = O.OracleOptimizer(model, 1e-3)
    for a, b in ((0, 2), (2, 6), (6, 9)):
        ((model(x[a:b]) - target[a:b]).square().sum() / 9).backward()
    before = model.proj.weight.detach().clone()
    opt.step()
    st = opt.st(model.proj.weight)
    torch.testing.assert_close(st["a_ema"], x.square().mean(0))
    torch.testing.assert_close(st["b_ema"], expect_b)
    assert st["a_count"] == st["b_count"] == 0
    assert not torch.equal(before, model.proj.weight)


def test_planted_ema_slip_is_caught():
    st = {"a_sum": torch.tensor([2.0, 4.0]), "a_count": 2, "a_ema": torch.tensor([1.0, 1.0])}
    O.finish_a(st, rank_one=False)
    # 0.97*1 + 0.03*(sum/count) in closed form
    torch.testing.assert_close(st["a_ema"], torch.tensor([0.97 + 0.03 * 1.0, 0.97 + 0.03 * 2.0]))
    st2 = {"a_sum": torch.tensor([2.0, 4.0]), "a_count": 2, "a_ema": torch.tensor([1.0, 1.0])}
    O.finish_a(st2, rank_one=False, beta=0.9)  # a wrong beta must not pass the same check
    with pytest.raises(AssertionError):
        torch.testing.assert_close(st2["a_ema"], st["a_ema"])


@pytest.mark.parametrize("rank_one", [True, False])
@pytest.mark.parametrize("shape", [(4, 4), (7, 3), (3, 7)])
def test_update_norm_is_sqrt_rows(rank_one, shape):
    # tests/test_optimizer.py:215-237
    torch.manual_seed(15)
    rows, cols = shape
    model = Proj(rows, cols)
    opt = O.OracleOptimizer(model, 1e-3, rank_one_a=rank_one)
    before = model.proj.weight.detach().clone()
    (model(torch.randn(12, cols)) - torch.randn(12, rows)).square().mean().backward()
    opt.step()
    norm = (model.proj.weight.detach() - before).norm() / 1e-3
    assert abs(norm.item() - rows ** .5) <= 2e-5 * rows ** .5 + 2e-5


def test_state_resume_matches_continuous():
    # tests/test_optimizer.py:95-113, on the oracle's state dict.
    torch.manual_seed(11)
    a = nn.Sequential(nn.Linear(4, 5), nn.Tanh(), nn.Linear(5, 2))
    b = copy.deepcopy(a)
    oa = O.OracleOptimizer(a, 2e-3)
    x, y = torch.randn(8, 4), torch.randn(8, 2)

    def one(model, opt):
        for p in model.parameters():
            p.grad = None
        (model(x) - y).square().mean().backward()
        opt.step()
    one(a, oa)
    ob = O.OracleOptimizer(b, 2e-3)
    b.load_state_dict(a.state_dict())
    ids_a = {n: id(p) for n, p in a.named_parameters()}
    ids_b = {n: id(p) for n, p in b.named_parameters()}
    ob.state = {ids_b[n]: copy.deepcopy(oa.state[ids_a[n]]) for n in ids_a if ids_a[n] in oa.state}
    one(a, oa)
    one(b, ob)
    for pa, pb in zip(a.parameters(), b.parameters()):
        torch.testing.assert_close(pa, pb)


def test_zero_signal_finite():
    # tests/test_optimizer.py:116-137
    model = Proj(3, 4)
    opt = O.OracleOptimizer(model, 1e-3)
    (model(torch.zeros(6, 4)) * 0).sum().backward()
    opt.step()
    assert torch.isfinite(model.proj.weight).all()
    st = opt.st(model.proj.weight)
    for k in ("a_ema", "a_mean_ema", "b_ema"):
        assert torch.isfinite(st[k]).all()


# -------------------------------------------- compensated-BF16 model ---
def _wide_range(seed, shape):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * torch.exp(torch.empty(*shape).uniform_(-8, 8, generator=g))).float()


def test_split_halves_are_bf16_and_keep_16_bits():
    t = _wide_range(1, (4096,))
    hi, lo = O._split(t)
    assert torch.equal(hi, hi.bfloat16().float()) and torch.equal(lo, lo.bfloat16().float())
    assert bool(((t.double() - hi.double() - lo.double()).abs() <= 2.0 ** -16 * t.double().abs()).all())
    # hi alone keeps only 8 bits: the bound must be the lo half's doing.
    assert not bool(((t.double() - hi.double()).abs() <= 2.0 ** -16 * t.double().abs()).all())


def _bound(a, b):
    return a.double().abs() @ b.double().abs()


def test_mm_comp_is_within_2_to_minus_16_of_the_exact_product():
    # reproduction/odl/ops/bf16_compensated_mm_fast.py:60-66: three products
    # of the hi/lo halves.  Each element of the result lies within
    # 2^-16 (|a||b|) of the float64 product; a plain BF16 product does not.
    a, b = _wide_range(2, (40, 64)), _wide_range(3, (64, 30))
    exact = a.double() @ b.double()
    err = (O._mm_comp(a, b).double() - exact).abs()
    assert bool((err <= 2.0 ** -16 * _bound(a, b)).all())
    plain = (O._mm_comp(a, b, comp=False).double() - exact).abs()
    assert not bool((plain <= 2.0 ** -16 * _bound(a, b)).all())
    assert bool((plain <= 2.0 ** -7 * _bound(a, b)).all())


def test_planted_dropped_correction_product_is_caught():
    a, b = _wide_range(4, (40, 64)), _wide_range(5, (64, 30))
    ah, al = O._split(a)
    bh, bl = O._split(b)
    dropped = (ah.double() @ bh.double() + ah.double() @ bl.double()).float()  # lo*hi missing
    err = (dropped.double() - a.double() @ b.double()).abs()
    assert not bool((err <= 2.0 ** -16 * _bound(a, b)).all())


RECIPES = [dict(comp_stages=0), dict(comp_stages=1), dict(comp_stages=3), dict(comp_stages=5),
           dict(mask=0x15), dict(fp16_stages=(3, 4, 5)), dict(fp16_stages=(2, 3, 4, 5))]


@pytest.mark.parametrize("recipe", RECIPES, ids=lambda r: "-".join(f"{k}{v}" for k, v in r.items()))
@pytest.mark.parametrize("shape", [(2, 7, 3), (2, 3, 7), (1, 40, 64)])
def test_comp_model_without_rounding_is_the_exact_map(monkeypatch, shape, recipe):
    # With the BF16 and FP16 roundings replaced by the identity every stored
    # operand is exact (lo = 0) and the float64 model must reduce to the SVD
    # closed form: this pins its scaling, orientation, stage order and the
    # (b/c) G term in every recipe.
    monkeypatch.setattr(O, "_bf16", lambda t: t)
    monkeypatch.setattr(O, "_f16", lambda t: t)
    torch.manual_seed(17)
    x = torch.randn(*shape, dtype=torch.float64)
    torch.testing.assert_close(O.s8_comp_bf16_model(x, **recipe), O.s8_svd(x), atol=1e-10, rtol=1e-9)
    # A planted slip (the stage coefficients in the wrong order) is caught.
    slipped = O.s8_comp_bf16_model(x, coefficients=O.S8_COEFFICIENTS[::-1], **recipe)
    assert not torch.allclose(slipped, O.s8_svd(x), atol=1e-3)


def test_mm_f16_is_within_2_to_minus_10_of_the_exact_product():
    # FP16 operands (11-bit significands) and a wide accumulator: every
    # element within 2^-10 (|a||b|) of the float64 product, and finer than a
    # plain BF16 product on the same (normal-range) operands.
    g = torch.Generator().manual_seed(9)
    a = torch.randn(40, 64, generator=g) * torch.exp(torch.empty(40, 64).uniform_(-3, 3, generator=g))
    b = torch.randn(64, 30, generator=g) * torch.exp(torch.empty(64, 30).uniform_(-3, 3, generator=g))
    exact = a.double() @ b.double()
    e16 = (O._mm_f16(a, b).double() - exact).abs()
    assert bool((e16 <= 2.0 ** -10 * _bound(a, b)).all())
    ebf = (O._mm_comp(a, b, comp=False).double() - exact).abs()
    assert e16.norm() < ebf.norm() / 4


def test_comp_bf16_model_is_within_gate_on_cfg2_like_input():
    # Budget of the rounding model against the FP32 oracle on an input with
    # log-uniform row/column scales: all five stages compensated sit far
    # inside the 1e-2 gate; with none compensated the error is much larger.
    from sandmuon_amd.workloads import s8_cfg2_batch
    x = s8_cfg2_batch(7, 1, 96, 160)
    ref = O.s8(x).double()
    err = lambda y: ((y.double() - ref).norm() / ref.norm()).item()
    full, none = err(O.s8_comp_bf16_model(x, 5)), err(O.s8_comp_bf16_model(x, 0))
    assert full < 1e-3, full
    assert none > 10 * full, (none, full)
    # the mixed recipe (compensated stages 1-2, FP16 stages 3-5) lies between
    mixed = err(O.s8_comp_bf16_model(x, fp16_stages=(3, 4, 5)))
    assert full < mixed < none and mixed < 5e-3, (full, mixed, none)


def _steep(n, p, seed):
    """An n x n matrix with singular values i^-p (a low-rank training
    gradient's shape) and random singular vectors."""
    g = torch.Generator().manual_seed(seed)
    u, _ = torch.linalg.qr(torch.randn(n, n, generator=g, dtype=torch.float64))
    v, _ = torch.linalg.qr(torch.randn(n, n, generator=g, dtype=torch.float64))
    return ((u * torch.arange(1, n + 1, dtype=torch.float64) ** -p) @ v.T).float()


@pytest.mark.parametrize("p", [1.5, 2.0])
def test_mixed_model_on_steep_spectra(p):
    # The rounding model on steeply decaying spectra: FP16 rounding of the
    # iterate lands in the small singular directions that the remaining
    # stages amplify.  With FP16 from stage 2 the error reaches the 1e-2
    # gate at p = 2; the mixed recipe (stage 2 compensated, FP16 stages 3-5)
    # stays at a third of it, an order of magnitude above the fully
    # compensated recipe.
    x = _steep(384, p, 7)
    ref = O.s8(x).double()
    err = lambda y: ((y.double() - ref).norm() / ref.norm()).item()
    comp = err(O.s8_comp_bf16_model(x))
    mixed = err(O.s8_comp_bf16_model(x, fp16_stages=(3, 4, 5)))
    early = err(O.s8_comp_bf16_model(x, fp16_stages=(2, 3, 4, 5)))
    assert comp < 1e-3 and mixed > 3 * comp and mixed < 3.5e-3, (comp, mixed)
    assert early > 2 * mixed, (mixed, early)
    if p == 2.0:
        assert early > 1e-2, early
