"""Parameter dtypes and layouts, and steps with more shape classes than one
S8 launch holds.

* bf16 / fp16 parameters: the reference keeps FP32 momentum and AdamW state
  and writes direction.to(parameter.dtype) (sandmuon/optimizer.py:245,
  :270-281, :315).  Compared with the CPU oracle, which does the same in the
  parameter dtype: FP32 state to 1e-6, parameters to two units in the last
  place of their dtype at the scale of the update's operands.  The two
  sides legitimately differ there: on the CPU, torch rounds the `alpha` of
  add_(d, alpha=-lr) to the tensor dtype before its FP32 multiply-add; on a
  GPU (torch's and this build's) alpha stays FP32.  The direction's own
  rounding to the dtype flips wherever the two directions straddle a
  rounding boundary.
* Layouts: a matrix parameter stored transposed is refused (the matrix
  kernels read row-major [rows, cols]); a channels_last Conv2d weight in the
  AdamW group is updated in its own layout, with a gradient in the same or
  in another layout, to 1e-6 of the oracle's AdamW.
* More than 8 distinct oriented shapes (10 here, half of them transposed
  parameters) split the step into several S8 plans over one workspace; both
  S8 modes against the oracle at the direction gates, with a bad gradient
  layout (a converted temporary per matrix) so that the temporaries must
  outlive their loop.
"""
import copy

import pytest
import torch
from torch import nn

from oracle import sandmuon_oracle as O
from sandmuon_amd import DiagonalWeightedPE, RankOneAWeightedPE
from sandmuon_amd.workloads import GPT, GPT_TINY, transformer_filter

from test_gpu_optimizer import DIR_TOL, Pair, check_directions, rel

pytestmark = pytest.mark.gpu


def ulp_close(a, b, before, dtype, upd_tol=0.0):
    """Elements where |a - b| exceeds one unit in the last place of dtype at
    the scale of the update's operands (the parameter before and after):
    where p and lr*d nearly cancel, a fused and an unfused multiply-add
    differ by far more than one ulp of the small result, but not of p.
    upd_tol adds that fraction of the element's update |before - b| (the
    mixed S8 mode's directions are ~2e-3 from the FP32 map, which on a
    near-zero weight is more than two ulps of it)."""
    a, b, before = (t.detach().float().cpu() for t in (a, b, before))
    scale = torch.maximum(torch.maximum(a.abs(), b.abs()), before.abs())
    bad = (a - b).abs() > 2 * torch.finfo(dtype).eps * scale + upd_tol * (before - b).abs()
    return int(bad.sum()), a.numel()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mode", ["fp32", "comp_bf16", "mixed"])
def test_low_precision_parameters_match_the_oracle(device, dtype, mode):
    torch.manual_seed(41)
    model = GPT(GPT_TINY)
    model.init_weights(41)
    model = model.to(dtype)
    lr = 3e-3
    pair = Pair(device, model, RankOneAWeightedPE, mode, lr, transformer_filter)
    g = torch.Generator().manual_seed(42)
    batches = [(torch.randint(0, GPT_TINY.vocab, (3, GPT_TINY.ctx), generator=g),
                torch.randint(0, GPT_TINY.vocab, (3, GPT_TINY.ctx), generator=g)) for _ in range(2)]
    loss = lambda m, x, y: m(x, y) / 2
    for _ in range(2):
        before, after_g, after_c = pair.step(batches, loss)
        for n, p in after_g.items():
            assert p.dtype == dtype
            bad, total = ulp_close(p, after_c[n], before[n], dtype, 5e-2 if mode == "mixed" else 0.0)
            assert bad <= max(1, total // 200), (n, bad, total)
        for n in pair.opt.named_matrices:
            dg = (before[n] - after_g[n]).float().cpu()
            dc = (before[n].cpu() - after_c[n]).float()
            # the updates agree up to the rounding of the parameter dtype
            # (one ulp of p is a few percent of a 1e-3-scale update)
            assert rel(dg, dc) <= 5e-2, (n, rel(dg, dc))
        for p_g, p_c in zip(pair.opt.param_groups[-1]["params"], pair.ora.aux):
            gs, cs = pair.opt.state[p_g], pair.ora.st(p_c)
            assert gs["exp_avg"].dtype == torch.float32
            assert rel(gs["exp_avg"], cs["exp_avg"]) <= 1e-6 and rel(gs["exp_avg_sq"], cs["exp_avg_sq"]) <= 1e-6
        for p in pair.opt.named_matrices.values():
            assert pair.opt.state[p]["momentum_buffer"].dtype == torch.float32
    pair.close()


def test_matrix_parameter_stored_transposed_is_refused(device):
    model = nn.Sequential(nn.Linear(6, 4)).to(device)
    model[0].weight = nn.Parameter(torch.randn(6, 4, device=device).t())  # [4, 6] with strides (1, 4)
    with pytest.raises(ValueError, match="row-major contiguous"):
        RankOneAWeightedPE(model, 1e-3)


class ConvNet(nn.Module):
    def __init__(self):
        super().__init__()
        self.conv = nn.Conv2d(3, 8, 3, padding=1)
        self.proj = nn.Linear(8, 5)

    def forward(self, x):
        return self.proj(torch.relu(self.conv(x)).mean((2, 3)))


@pytest.mark.parametrize("grad_layout", ["same", "contiguous"])
def test_channels_last_auxiliary_parameter(device, grad_layout):
    torch.manual_seed(43)
    model = ConvNet().to(device).to(memory_format=torch.channels_last)
    w = model.conv.weight
    assert not w.is_contiguous() and w.is_contiguous(memory_format=torch.channels_last)
    cpu = copy.deepcopy(model).cpu()
    lr = 1e-2
    opt = RankOneAWeightedPE(model, lr)
    ora = O.OracleOptimizer(cpu, lr, rank_one_a=True, hooks=False)
    x = torch.randn(4, 3, 6, 6)
    y = torch.randn(4, 5)
    for _ in range(2):
        opt.zero_grad(set_to_none=True)
        (model(x.to(device).contiguous(memory_format=torch.channels_last)) - y.to(device)).square().mean().backward()
        if grad_layout == "contiguous":
            w.grad = w.grad.contiguous()
            assert w.grad.stride() != w.stride()
        with torch.no_grad():
            for pg, pc in zip(model.parameters(), cpu.parameters()):
                pc.copy_(pg.detach().cpu())
                pc.grad = pg.grad.detach().cpu().clone()
        opt.step()
        # the oracle's AdamW on the auxiliary parameters (its matrix step
        # needs hook inputs and is not compared here)
        with torch.no_grad():
            for p in ora.aux:
                O.adamw(p, p.grad.float(), ora.st(p), lr * .1)
        torch.cuda.synchronize()
        assert w.is_contiguous(memory_format=torch.channels_last)
        assert rel(w, cpu.conv.weight) <= 1e-6
        assert rel(model.conv.bias, cpu.conv.bias) <= 1e-6
        st = opt.state[w]
        assert st["exp_avg"].stride() == w.stride()
        assert rel(st["exp_avg"], ora.st(cpu.conv.weight)["exp_avg"]) <= 1e-6
    opt.close()


class Branches(nn.Module):
    """Ten independent Linear layers of ten distinct oriented shapes (every
    other one a transposed parameter, rows > cols), each fed a slice of one
    full-rank input, so that every gradient has full rank.  (A chain of such
    layers would feed the 100-wide layer after the 24-wide one activations
    near a 24-dimensional manifold, and a rank-deficient gradient cannot be
    held to the 1e-4 FP32 gate: the polar map amplifies rounding in its null
    space.)"""
    SHAPES = ((96, 64), (40, 96), (130, 40), (72, 130), (200, 72), (24, 200), (100, 24), (56, 100), (150, 56),
              (32, 150))

    def __init__(self):
        super().__init__()
        self.layers = nn.ModuleList(nn.Linear(i, o) for o, i in self.SHAPES)

    def forward(self, x):
        return torch.cat([layer(x[:, :layer.in_features]) for layer in self.layers], 1)


@pytest.mark.parametrize("opt_cls", [RankOneAWeightedPE, DiagonalWeightedPE])
@pytest.mark.parametrize("mode", ["fp32", "comp_bf16", "mixed"])
def test_more_than_eight_shape_classes(device, opt_cls, mode):
    torch.manual_seed(44)
    model = Branches()
    shapes = {tuple(sorted(l.weight.shape)) for l in model.layers}
    assert len(shapes) == 10 and sum(l.weight.shape[0] > l.weight.shape[1] for l in model.layers) == 5
    lr = 1e-3
    pair = Pair(device, model, opt_cls, mode, lr)
    g = torch.Generator().manual_seed(45)
    out = sum(o for o, _ in Branches.SHAPES)
    batches = [(torch.randn(2048, 200, generator=g) + torch.randn(200, generator=g),
                torch.randn(2048, out, generator=g)) for _ in range(2)]
    loss = lambda m, x, y: (m(x) - y).square().mean() / 2

    def transposed_grads(m):
        # same values, column-major strides: step() makes one contiguous
        # temporary per matrix
        for layer in m.layers:
            layer.weight.grad = layer.weight.grad.t().contiguous().t()
            assert not layer.weight.grad.is_contiguous()

    hist = [pair.step(batches, loss, prepare=transposed_grads) for _ in range(2)]
    worst = check_directions(hist, pair.opt, lr, mode)
    print(f"10 shape classes {opt_cls.__name__} {mode}: worst direction rel err {worst:.3e}")
    assert worst <= DIR_TOL[mode]
    pair.close()
