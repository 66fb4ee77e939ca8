"""The reference's own test intents (tests/test_optimizer.py), run on this
build's API on the GPU: the module-level helpers against dense oracles in
float64 (the reference's dtype for them) and against the CPU oracle in
float32, zero signal in both variants, the closure under enable_grad,
statistics over uneven microbatches, the update norm of every aspect, q/k/v
sharing, and the RuntimeErrors of sandmuon/optimizer.py:184-185 and
:211-212.

Gates: the float64 dense-oracle identities at the reference's 1e-10; the
float32 helpers within 1e-5 (relative Frobenius) of the float32 oracle;
statistics at the north star's 1e-6."""
import pytest
import torch
from torch import nn

from oracle import sandmuon_oracle as O
from sandmuon_amd import DiagonalWeightedPE, RankOneAWeightedPE
from sandmuon_amd.optimizer import (_graft_direction, diagonal_inverse_sqrt, rank1_inverse_sqrt, rank1_mapback,
                                    rank1_whiten)

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-300)).item()


def _dense_whitener(second, mean):
    inverse, z, coefficient = rank1_inverse_sqrt(second, mean)
    correction = torch.eye(second.numel(), dtype=second.dtype) + coefficient * torch.outer(z, z)
    return correction @ torch.diag(inverse)


def test_rank_one_whitener_matches_dense_covariance_oracle(device):
    # tests/test_optimizer.py:24-43, float64 on the GPU helpers.
    torch.manual_seed(7)
    x = torch.randn(500, 6, dtype=torch.float64) + torch.randn(6, dtype=torch.float64)
    second, mean = x.square().mean(0), x.mean(0)
    inverse, z, coefficient = rank1_inverse_sqrt(second, mean)
    assert inverse.dtype == z.dtype == coefficient.dtype == torch.float64 and coefficient.shape == ()
    w = _dense_whitener(second, mean)
    covariance = torch.diag(second - mean.square()) + torch.outer(mean, mean)
    torch.testing.assert_close(w @ (covariance / second.mean()) @ w.T, torch.eye(6, dtype=torch.float64),
                               atol=1e-10, rtol=1e-10)
    source = torch.randn(2, 6, 4, dtype=torch.float64)
    right = rank1_inverse_sqrt(second[:4], mean[:4])
    actual = rank1_whiten(source, (inverse, z, coefficient), right)
    assert actual.dtype == torch.float64 and actual.device.type == "cpu"
    dense_right = _dense_whitener(second[:4], mean[:4])
    expected = torch.stack([w @ item @ dense_right.T for item in source])
    torch.testing.assert_close(actual, expected, atol=1e-10, rtol=1e-10)


def test_mapback_applies_rank_one_factors_then_diagonal(device):
    # tests/test_optimizer.py:46-54, float64.
    torch.manual_seed(8)
    q = torch.randn(5, 3, dtype=torch.float64)
    li, lz, lc = rank1_inverse_sqrt(torch.rand(5, dtype=torch.float64) + .3, torch.randn(5, dtype=torch.float64) * .1)
    ri, rz, rc = rank1_inverse_sqrt(torch.rand(3, dtype=torch.float64) + .3, torch.randn(3, dtype=torch.float64) * .1)
    left = torch.eye(5, dtype=q.dtype) + lc * torch.outer(lz, lz)
    right = torch.eye(3, dtype=q.dtype) + rc * torch.outer(rz, rz)
    expected = torch.diag(li) @ left @ q @ right @ torch.diag(ri)
    torch.testing.assert_close(rank1_mapback(q, (li, lz, lc), (ri, rz, rc)), expected)


def _factors(n, seed, dtype=torch.float32):
    """Statistics as the hooks produce them: second >= mean^2, so every
    channel has a positive variance (a clamped one gives 1e3-scale factors
    whose rank-one term cancels in FP32)."""
    g = torch.Generator().manual_seed(seed)
    mean = torch.randn(n, generator=g, dtype=torch.float64) * .4
    second = mean.square() + torch.rand(n, generator=g, dtype=torch.float64) + .3
    return second.to(dtype), mean.to(dtype)


@pytest.mark.parametrize("shape", [(2, 6, 4), (1, 5, 3), (1, 768, 3072)])
def test_float32_helpers_match_the_oracle(device, shape):
    # The helpers reach smx_inverse_sqrt, smx_rank1_apply and smx_graft.
    b, r, c = shape
    g = torch.Generator().manual_seed(r * 31 + c)
    x = torch.randn(*shape, generator=g)
    ls, lm = _factors(r, 1)
    rs, rm = _factors(c, 2)
    got_l, want_l = rank1_inverse_sqrt(ls, lm), O.rank1_inverse_sqrt(ls, lm)
    got_r, want_r = rank1_inverse_sqrt(rs, rm), O.rank1_inverse_sqrt(rs, rm)
    for got, want in zip(got_l + got_r, want_l + want_r):
        assert got.dtype == torch.float32 and rel(got, want) <= F32_TOL
    assert rel(diagonal_inverse_sqrt(ls), O.diagonal_inverse_sqrt(ls)) <= F32_TOL
    lb = tuple(t.expand(b, *t.shape) if t.ndim else t.expand(b) for t in want_l)
    rb = tuple(t.expand(b, *t.shape) if t.ndim else t.expand(b) for t in want_r)
    whitened = rank1_whiten(x, want_l, want_r)
    assert rel(whitened, O.rank1_whiten(x, lb, rb)) <= F32_TOL
    mapped = rank1_mapback(x[0], want_l, want_r)
    assert rel(mapped, O.rank1_mapback(x[0], want_l, want_r)) <= F32_TOL
    grafted = _graft_direction(mapped, r)
    assert grafted.dtype == torch.float32
    # The graft's norm is summed in FP64 here; the reference's FP32 norm over
    # millions of elements is itself ~1e-5 off, so the scale is compared
    # with the oracle's graft in float64 of the oracle's mapped value.
    want_mapped = O.rank1_mapback(x[0], want_l, want_r)
    assert rel(grafted, O.graft_direction(want_mapped.double(), r)) <= F32_TOL
    assert abs(grafted.double().norm().item() - r ** .5) <= 1e-5 * r ** .5
    # float64 inputs graft in float32, as the reference's .float() does
    assert _graft_direction(mapped.double(), r).dtype == torch.float32


class Proj(nn.Module):
    def __init__(self, rows, cols, bias=False):
        super().__init__()
        self.proj = nn.Linear(cols, rows, bias=bias)

    def forward(self, x):
        return self.proj(x)


@pytest.mark.parametrize("opt_cls", [RankOneAWeightedPE, DiagonalWeightedPE])
@pytest.mark.parametrize("rows", [3, 16])
def test_zero_signal_remains_finite_with_a_zero_update(device, opt_cls, rows):
    # tests/test_optimizer.py:116-137 and :195-212.  With 16 rows the
    # reference's sqrt(rows)/FLT_MIN overflows and its update is NaN; here a
    # zero direction gives a zero update (documented divergence).
    model = Proj(rows, 4).to(device)
    before = model.proj.weight.detach().clone()
    opt = opt_cls(model, lr=1e-3)
    opt.zero_grad(set_to_none=True)
    (model(torch.zeros(6, 4, device=device)) * 0).sum().backward()
    opt.step()
    assert torch.equal(model.proj.weight.detach(), before)
    state = opt.state[model.proj.weight]
    keys = ("a_ema", "a_mean_ema", "b_ema") if opt_cls is RankOneAWeightedPE else ("a_ema", "b_ema")
    for key in keys:
        assert torch.isfinite(state[key]).all(), key
    assert torch.isfinite(diagonal_inverse_sqrt(torch.zeros(4))).all()
    opt.close()


def test_step_closure_runs_with_grad_enabled(device):
    # tests/test_optimizer.py:240-259 and sandmuon/optimizer.py:226-230.
    torch.manual_seed(16)
    model = nn.Sequential(nn.Linear(4, 5), nn.Tanh(), nn.Linear(5, 2)).to(device)
    opt = RankOneAWeightedPE(model, lr=1e-3)
    x, target = torch.randn(7, 4, device=device), torch.randn(7, 2, device=device)
    before = [p.detach().clone() for p in model.parameters()]
    seen = []

    def closure():
        seen.append(torch.is_grad_enabled())
        opt.zero_grad(set_to_none=True)
        loss = (model(x) - target).square().mean()
        loss.backward()
        return loss

    loss = opt.step(closure)
    assert seen == [True] and torch.isfinite(loss)
    assert all(not torch.equal(old, new) for old, new in zip(before, model.parameters()))
    assert all(p.grad is not None and torch.isfinite(p.grad).all() for p in model.parameters())
    opt.close()


def test_statistics_accumulate_over_uneven_microbatches(device):
    # tests/test_optimizer.py:57-85: a_ema = mean x^2 over the whole
    # effective batch, b_ema = the normalised analytic cotangent shape.
    torch.manual_seed(10)
    model = Proj(3, 4).to(device)
    x = torch.randn(9, 4, device=device)
    target = torch.randn(9, 3, device=device)
    with torch.no_grad():
        pred = model(x)
    expected_b = (2 * (pred - target) / x.shape[0]).square().mean(0)
    expected_b = expected_b / expected_b.mean()
    opt = RankOneAWeightedPE(model, lr=1e-3)
    opt.zero_grad(set_to_none=True)
    for start, end in ((0, 2), (2, 6), (6, 9)):
        ((model(x[start:end]) - target[start:end]).square().sum() / x.shape[0]).backward()
    before = model.proj.weight.detach().clone()
    opt.step()
    state = opt.state[model.proj.weight]
    assert rel(state["a_ema"], x.square().mean(0)) <= 1e-6
    assert rel(state["a_mean_ema"], x.mean(0)) <= 1e-6
    assert rel(state["b_ema"], expected_b) <= 1e-6
    assert state["a_count"] == state["b_count"] == 0
    assert not torch.equal(before, model.proj.weight)
    opt.close()


@pytest.mark.parametrize("opt_cls", [DiagonalWeightedPE, RankOneAWeightedPE])
@pytest.mark.parametrize("rows,cols", [(4, 4), (7, 3), (3, 7)])
def test_update_norm_is_sqrt_rows_for_every_aspect(device, opt_cls, rows, cols):
    # tests/test_optimizer.py:215-237
    torch.manual_seed(15)
    lr = 1e-3
    model = Proj(rows, cols).to(device)
    opt = opt_cls(model, lr=lr)
    x, target = torch.randn(12, cols, device=device), torch.randn(12, rows, device=device)
    before = model.proj.weight.detach().clone()
    (model(x) - target).square().mean().backward()
    opt.step()
    norm = ((model.proj.weight.detach() - before).double().norm() / lr).item()
    assert abs(norm - rows ** .5) <= 2e-5 * max(1.0, rows ** .5) + 2e-5
    opt.close()


def test_qkv_share_the_activation_statistic_of_q(device):
    # tests/test_optimizer.py:152-193
    class Attention(nn.Module):
        def __init__(self):
            super().__init__()
            self.q_proj = nn.Linear(4, 4, bias=False)
            self.k_proj = nn.Linear(4, 4, bias=False)
            self.v_proj = nn.Linear(4, 4, bias=False)

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.attn = Attention()
            self.cross_attn = Attention()

        def forward(self, x):
            return sum(m(x) for a in (self.attn, self.cross_attn) for m in (a.q_proj, a.k_proj, a.v_proj))

    class Model(nn.Module):
        def __init__(self):
            super().__init__()
            self.transformer = nn.Module()
            self.transformer.h = nn.ModuleList([Block()])

        def forward(self, x):
            return self.transformer.h[0](x)

    torch.manual_seed(14)
    model = Model().to(device)
    block = model.transformer.h[0]
    opt = RankOneAWeightedPE(model, lr=1e-3)
    assert opt.a_sources[id(block.attn.k_proj.weight)] is block.attn.q_proj.weight
    assert opt.a_sources[id(block.cross_attn.k_proj.weight)] is block.cross_attn.k_proj.weight
    x = torch.randn(5, 4, device=device)
    opt.zero_grad(set_to_none=True)
    model(x).square().mean().backward()
    opt.step()
    assert rel(opt.state[block.attn.q_proj.weight]["a_ema"], x.square().mean(0)) <= 1e-6
    assert "a_ema" not in opt.state[block.attn.k_proj.weight]
    opt.close()


@pytest.mark.parametrize("opt_cls", [RankOneAWeightedPE, DiagonalWeightedPE])
def test_missing_activation_statistics_raise(device, opt_cls):
    # sandmuon/optimizer.py:184-185: a step after an eval-mode forward (the
    # hooks take nothing) has no activation statistics.
    model = Proj(3, 4).to(device)
    opt = opt_cls(model, lr=1e-3)
    model.eval()
    model(torch.randn(6, 4, device=device)).square().sum().backward()
    before = model.proj.weight.detach().clone()
    with pytest.raises(RuntimeError, match="Missing activation statistics: proj.weight"):
        opt.step()
    assert torch.equal(model.proj.weight.detach(), before)
    opt.close()


@pytest.mark.parametrize("opt_cls", [RankOneAWeightedPE, DiagonalWeightedPE])
def test_mismatched_cotangent_counts_raise(device, opt_cls):
    # sandmuon/optimizer.py:211-212: a second forward without its backward
    # leaves the cotangent count short of the activation count.
    model = Proj(3, 4).to(device)
    opt = opt_cls(model, lr=1e-3)
    model(torch.randn(6, 4, device=device)).square().sum().backward()
    model(torch.randn(5, 4, device=device))
    with pytest.raises(RuntimeError, match=r"Missing or mismatched cotangent statistics: proj.weight; "
                                           r"expected 11, got 6"):
        opt.step()
    opt.close()
