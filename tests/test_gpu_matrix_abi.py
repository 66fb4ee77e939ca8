"""The matrix step and AdamW through the C ABI as a non-torch host calls
them, and the optimizer on shapes that take the kernels' scalar paths.

* bf16/f16 gradients (smx_matrix_desc.grad_dtype, smx_adamw_desc.grad_dtype):
  torch keeps fp32 gradients for fp32 parameters, so only another host
  reaches these paths.  The momentum and AdamW are elementwise and must equal
  the fp32-gradient run on the same (exactly widened) values bit for bit;
  the update direction, whose row sums run in another order on the scalar
  path, to 1e-5 (fp32 mode) and 1e-4 (comp_bf16 mode).
* odd shapes (columns not a multiple of 4, transposed parameters, sizes far
  from the 256 padding) through the whole optimizer against the CPU oracle,
  at the north-star gates;
* seeded random shapes (widths 1-900, edge sizes around the padding and the
  tiles, more distinct shapes than one S8 plan takes) the same way.
"""
import math

import pytest
import torch
from torch import nn

from sandmuon_amd import DiagonalWeightedPE, RankOneAWeightedPE, _native

from test_gpu_optimizer import check_aux, check_directions, rel, run_pair

pytestmark = pytest.mark.gpu


def _factors(rows, cols, seed, device):
    g = torch.Generator().manual_seed(seed)
    inv_row = torch.rand(rows, generator=g) + 0.5
    inv_col = torch.rand(cols, generator=g) + 0.5
    z = torch.randn(cols, generator=g) * 0.3
    rho = math.sqrt(1.0 + float((z.double() ** 2).sum()))
    kappa = torch.tensor([-1.0 / (rho * (rho + 1.0))])
    return [t.float().to(device) for t in (inv_row, inv_col, z, kappa)]


@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("gdt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(96, 64), (64, 96), (37, 53), (130, 7)])
def test_matrix_step_low_precision_gradients(device, mode, gdt, shape):
    rows, cols = shape
    inv_row, inv_col, z, kappa = _factors(rows, cols, rows * cols, device)
    g = torch.Generator().manual_seed(rows + cols)
    grad_lp = (torch.randn(rows, cols, generator=g) * 1e-2).to(gdt).to(device)
    mom0 = torch.randn(rows, cols, generator=g) * 1e-2
    w0 = torch.randn(rows, cols, generator=g) * 0.02
    lr = 1e-2

    def run(grad):
        w, m = w0.clone().to(device), mom0.clone().to(device)
        d = _native.MatrixDesc(param=w.data_ptr(), grad=grad.data_ptr(), momentum=m.data_ptr(),
                               inv_row=inv_row.data_ptr(), inv_col=inv_col.data_ptr(), z=z.data_ptr(),
                               kappa=kappa.data_ptr(), rows=rows, cols=cols, lr=lr, momentum_beta=.8,
                               grad_dtype=_native.dtype_code(grad.dtype))
        ws = torch.empty(_native.matrix_step_workspace_bytes([shape], mode), dtype=torch.uint8, device=device)
        _native.matrix_step([d], mode, ws)
        torch.cuda.synchronize()
        return w, m

    w_lp, m_lp = run(grad_lp)
    w_32, m_32 = run(grad_lp.float().contiguous())
    assert torch.equal(m_lp, m_32)
    d_lp = (w0.to(device) - w_lp) / lr
    d_32 = (w0.to(device) - w_32) / lr
    # comp_bf16 rounds the iterate to 16-17 bits in every stage, so a
    # last-bit difference in the whitening row sums moves it by a few 1e-5;
    # the mixed mode's FP16 stages round it to 11 bits
    assert rel(d_lp, d_32) <= (1e-5 if mode == 0 else 1e-4 if mode == 1 else 2e-3)
    # the graft: ||direction|| = sqrt(rows)
    assert abs(d_lp.double().norm().item() - math.sqrt(rows)) <= 1e-4 * math.sqrt(rows)


@pytest.mark.parametrize("gdt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("sizes", [[1000, 4096, 3], [50257 * 3, 768, 1]])
def test_adamw_low_precision_gradients(device, gdt, sizes):
    g = torch.Generator().manual_seed(sum(sizes))
    params = [torch.randn(n, generator=g).to(device) for n in sizes]
    grads = [(torch.randn(n, generator=g) * 1e-3).to(gdt).to(device) for n in sizes]

    def run(gs):
        ps = [p.clone() for p in params]
        m = [torch.zeros_like(p) for p in params]
        v = [torch.zeros_like(p) for p in params]
        for step in (1, 2):
            descs, off = [], 0
            for p, gr, ea, es in zip(ps, gs, m, v):
                descs.append(_native.AdamwDesc(param=p.data_ptr(), grad=gr.data_ptr(), exp_avg=ea.data_ptr(),
                                               exp_avg_sq=es.data_ptr(), n=p.numel(), offset=off,
                                               bias1=1 - .9 ** step, bias2=1 - .999 ** step,
                                               grad_dtype=_native.dtype_code(gr.dtype)))
                off += p.numel()
            _native.adamw(descs, off, 1e-3, .9, .999, 1e-8, .01, device)
        torch.cuda.synchronize()
        return ps, m, v

    a = run(grads)
    b = run([gr.float() for gr in grads])
    for xs, ys in zip(a, b):
        for x, y in zip(xs, ys):
            assert torch.equal(x, y)


class Chain(nn.Module):
    """Linears of odd widths: 53 -> 37 -> 130 -> 7 -> 300 -> 5 (two of them
    transposed in the S8 map, every column count but one off a multiple of 4)."""

    def __init__(self):
        super().__init__()
        dims = [53, 37, 130, 7, 300, 5]
        self.layers = nn.ModuleList([nn.Linear(a, b) for a, b in zip(dims, dims[1:])])

    def forward(self, x):
        for k, layer in enumerate(self.layers):
            x = layer(x)
            if k + 1 < len(self.layers):
                x = torch.tanh(x)
        return x


@pytest.mark.parametrize("mode", ["fp32", "comp_bf16", "mixed"])
def test_odd_shapes_through_the_optimizer(device, tile_policy, mode):
    torch.manual_seed(41)
    model = Chain()
    g = torch.Generator().manual_seed(42)
    batches = [(torch.randn(4, 64, 53, generator=g) + 0.2, torch.randn(4, 64, 5, generator=g)) for _ in range(2)]
    loss = lambda m, x, y: (m(x) - y).square().mean() / 2
    hist, opt, ora = run_pair(device, model, batches, loss, RankOneAWeightedPE, mode, 1e-2, steps=2)
    assert len(opt.named_matrices) == 5
    worst = check_directions(hist, opt, 1e-2, mode)
    print(f"odd shapes {mode} tiles {tile_policy}: worst direction rel err {worst:.3e}")
    check_aux(hist, opt, ora)


class WideBranches(nn.Module):
    """Linears whose parameter rows take each path of the whiten kernel:
    in-widths 1000 and 2048 are taken by 2 and 4 waves per row with 2
    float4 per lane kept in registers (blocks of 4 row groups, 44 and 48
    rows: padding rows in the last block), 4096 and 4100 are wider and
    re-read g and m'; 64 -> 700 is a transposed parameter with one kept
    chunk, 1100 -> 1300 a transposed one whose 1100 columns re-read.  The batches hold more samples (4096) than the widest
    parameter has rows or columns: with fewer, the gradients of the 1100 x
    1300 parameter are rank-deficient, and the polar map of a rank-deficient
    matrix amplifies the rounding in its null space (two FP32 evaluations of
    such a matrix already differ by about 1.2e-4), which no FP32 gate can
    hold to 1e-4."""

    WIDTHS = [(1000, 44), (2048, 48), (4096, 40), (4100, 36), (64, 700), (1100, 1300)]

    def __init__(self):
        super().__init__()
        self.layers = nn.ModuleList([nn.Linear(a, b) for a, b in self.WIDTHS])

    def forward(self, x):
        parts = torch.split(x, [a for a, _ in self.WIDTHS], dim=-1)
        return torch.cat([torch.tanh(layer(p)) for layer, p in zip(self.layers, parts)], dim=-1)


@pytest.mark.parametrize("mode", ["fp32", "comp_bf16", "mixed"])
def test_wide_rows_through_the_optimizer(device, tile_policy, mode):
    torch.manual_seed(43)
    model = WideBranches()
    g = torch.Generator().manual_seed(44)
    d_in, d_out = sum(a for a, _ in WideBranches.WIDTHS), sum(b for _, b in WideBranches.WIDTHS)
    batches = [(torch.randn(4, 512, d_in, generator=g) * 0.5 + 0.1, torch.randn(4, 512, d_out, generator=g) * 0.5)
               for _ in range(2)]
    loss = lambda m, x, y: (m(x) - y).square().mean() / 2
    hist, opt, ora = run_pair(device, model, batches, loss, RankOneAWeightedPE, mode, 1e-2, steps=2)
    assert len(opt.named_matrices) == 6
    worst = check_directions(hist, opt, 1e-2, mode)
    print(f"wide rows {mode} tiles {tile_policy}: worst direction rel err {worst:.3e}")
    check_aux(hist, opt, ora)


class RandomBranches(nn.Module):
    """Parallel Linears of seeded random widths, edge sizes included (1-3,
    around the 256-element padding and the 512 and 768 tiles): tall, wide and
    square matrices, transposed and not, more distinct shapes than one S8
    plan takes (so the step runs in groups over one workspace)."""

    def __init__(self, seed):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        edge = [1, 2, 3, 16, 255, 256, 257, 511, 512, 513, 767, 769]
        dims = []
        for k in range(14):
            pick = lambda: (edge[int(torch.randint(0, len(edge), (1,), generator=g))] if k % 2 == 0
                            else int(torch.randint(1, 901, (1,), generator=g)))
            dims.append((pick(), pick()))
        self.widths = dims
        self.layers = nn.ModuleList([nn.Linear(a, b) for a, b in dims])

    def forward(self, x):
        parts = torch.split(x, [a for a, _ in self.widths], dim=-1)
        return torch.cat([torch.tanh(layer(p)) for layer, p in zip(self.layers, parts)], dim=-1)


@pytest.mark.parametrize("mode", ["fp32", "comp_bf16", "mixed"])
@pytest.mark.parametrize("seed,opt_cls", [(7, RankOneAWeightedPE), (8, RankOneAWeightedPE), (9, DiagonalWeightedPE)])
def test_random_shapes_through_the_optimizer(device, mode, seed, opt_cls):
    torch.manual_seed(seed)
    model = RandomBranches(seed)
    width_in = sum(a for a, _ in model.widths)
    width_out = sum(b for _, b in model.widths)
    g = torch.Generator().manual_seed(seed + 100)
    # more samples than any width, so every gradient has full rank
    batches = [(torch.randn(2048, width_in, generator=g) + 0.1, torch.randn(2048, width_out, generator=g))
               for _ in range(2)]
    loss = lambda m, x, y: (m(x) - y).square().mean() / 2
    hist, opt, ora = run_pair(device, model, batches, loss, opt_cls, mode, 1e-2, steps=2)
    shapes = {tuple(sorted(p.shape)) for p in opt.named_matrices.values()}
    assert len(opt.named_matrices) == 14 and len(shapes) > 8, model.widths
    worst = check_directions(hist, opt, 1e-2, mode)
    print(f"random shapes seed {seed} {opt_cls.__name__} {mode}: {model.widths}; worst direction rel err {worst:.3e}")
    check_aux(hist, opt, ora)


class Extremes(nn.Module):
    """Linears far from square: a 40 x 12000 weight (a Gram-space class
    whose Gram and apply run K = 12000), a 7000 x 33 weight (transposed, an
    odd column count on the scalar statistics path) and a 300 x 4100 one."""

    widths = [(12000, 40), (33, 7000), (4100, 300)]

    def __init__(self):
        super().__init__()
        self.layers = nn.ModuleList([nn.Linear(a, b) for a, b in self.widths])

    def forward(self, x):
        parts = torch.split(x, [a for a, _ in self.widths], dim=-1)
        return torch.cat([torch.tanh(layer(p)) for layer, p in zip(self.layers, parts)], dim=-1)


@pytest.mark.parametrize("mode", ["fp32", "comp_bf16", "mixed"])
def test_extreme_aspect_ratios_through_the_optimizer(device, mode):
    torch.manual_seed(11)
    model = Extremes()
    width_in = sum(a for a, _ in model.widths)
    width_out = sum(b for _, b in model.widths)
    g = torch.Generator().manual_seed(111)
    # 1024 samples: more than every matrix's smaller side, so each gradient has full rank
    batches = [(torch.randn(1024, width_in, generator=g) + 0.1, torch.randn(1024, width_out, generator=g))
               for _ in range(2)]
    loss = lambda m, x, y: (m(x) - y).square().mean() / 2
    hist, opt, ora = run_pair(device, model, batches, loss, RankOneAWeightedPE, mode, 1e-2, steps=2)
    assert sorted(tuple(p.shape) for p in opt.named_matrices.values()) == [(40, 12000), (300, 4100), (7000, 33)]
    worst = check_directions(hist, opt, 1e-2, mode)
    print(f"extreme aspect ratios {mode}: worst direction rel err {worst:.3e}")
    check_aux(hist, opt, ora)


class ManyBranches(nn.Module):
    """264 parallel Linears in four shape classes, half of them transposed
    parameters: the row kernels of the matrix step take at most 128 jobs per
    launch, so the whiten, the transposed whiten and both mapback kernels
    each run a second launch whose jobs (table entries 128 and up) are
    compared with the oracle like the first."""

    WIDTHS = [(32, 48), (48, 32), (64, 64), (24, 80)] * 66  # (in, out): weights 48x32 (transposed), 32x48, ...

    def __init__(self):
        super().__init__()
        self.layers = nn.ModuleList([nn.Linear(a, b) for a, b in self.WIDTHS])

    def forward(self, x):
        parts = torch.split(x, [a for a, _ in self.WIDTHS], dim=-1)
        return torch.cat([torch.tanh(layer(p)) for layer, p in zip(self.layers, parts)], dim=-1)


@pytest.mark.parametrize("mode", ["fp32", "comp_bf16", "mixed"])
def test_more_matrices_than_one_row_launch_takes(device, mode):
    torch.manual_seed(17)
    model = ManyBranches()
    d_in, d_out = sum(a for a, _ in ManyBranches.WIDTHS), sum(b for _, b in ManyBranches.WIDTHS)
    g = torch.Generator().manual_seed(18)
    # 256 samples: more than every matrix's smaller side (full-rank gradients)
    batches = [(torch.randn(256, d_in, generator=g) + 0.1, torch.randn(256, d_out, generator=g)) for _ in range(2)]
    loss = lambda m, x, y: (m(x) - y).square().mean() / 2
    hist, opt, ora = run_pair(device, model, batches, loss, RankOneAWeightedPE, mode, 1e-2, steps=2)
    mats = list(opt.named_matrices.values())
    flipped = sum(p.shape[0] > p.shape[1] for p in mats)
    assert len(mats) == 264 and flipped > 128 and len(mats) - flipped > 128
    worst = check_directions(hist, opt, 1e-2, mode)  # every matrix, so every job of both launches
    print(f"264 matrices ({flipped} transposed) {mode}: worst direction rel err {worst:.3e}")
    check_aux(hist, opt, ora)
