"""GPU parity of the statistics kernels (hooks + finish) against the oracle.

Gate (north star): statistics and EMA state within relative error 1e-6
(normwise ||gpu - ref|| / ||ref|| per vector).
"""
import pytest
import torch

from oracle import sandmuon_oracle as O
from sandmuon_amd import _native
from sandmuon_amd.workloads import stats_cfg3_tensor

pytestmark = pytest.mark.gpu

STATS_TOL = 1e-6


def rel(a, b):
    a = a.double().cpu()
    b = b.double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-300)).item()


def accumulate(x, n_slots=128, first=True):
    d = x.shape[-1]
    sq = torch.zeros(n_slots, d, device=x.device)
    fs = torch.zeros(n_slots, d, device=x.device) if first else None
    _native.stats_accumulate(x, sq, fs)
    tot_sq = torch.zeros(d, device=x.device)
    tot_f = torch.zeros(d, device=x.device) if first else None
    _native.stats_fold(tot_sq, sq, tot_f, fs)
    torch.cuda.synchronize()
    assert torch.count_nonzero(sq) == 0, "fold must zero the slots"
    return tot_sq, tot_f


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,cols", [(0, 8), (1, 4), (9, 4), (7, 5), (33, 100), (1000, 768), (16384, 768),
                                       (4096, 3072), (300, 24),
                                       (8192, 2048), (8192, 8192)])  # cfg5 hook shapes (8 x 1024 tokens)
def test_accumulate_matches_fp64_brute_force(device, dtype, rows, cols):
    x = stats_cfg3_tensor(rows * 7 + cols, rows, cols, dtype=dtype)
    sq, fs = accumulate(x.to(device))
    ref_sq = (x.double() ** 2).sum(0)
    ref_f = x.double().sum(0)
    if rows == 0:
        assert torch.count_nonzero(sq) == 0 and torch.count_nonzero(fs) == 0
        return
    assert rel(sq, ref_sq) <= STATS_TOL
    # sum(x) can cancel: compare normwise against the fp64 sum with an
    # absolute floor of the fp32 rounding of the sum of |x|.
    err = (fs.double().cpu() - ref_f).abs().max().item()
    bound = 1e-6 * x.double().abs().sum(0).max().item()
    assert err <= bound


def test_accumulate_over_microbatches_and_strided_rows(device):
    # Uneven microbatches (tests/test_optimizer.py:75 pattern) and a non-unit
    # row stride (a column slice of a wider tensor).
    full = stats_cfg3_tensor(5, 3000, 800, dtype=torch.float32)
    x = full[:, :768]
    sq = torch.zeros(128, 768, device=device)
    fs = torch.zeros(128, 768, device=device)
    xg = full.to(device)[:, :768]
    for a, b in ((0, 2), (2, 1500), (1500, 3000)):
        _native.stats_accumulate(xg[a:b], sq, fs)
    tot_sq = torch.zeros(768, device=device)
    tot_f = torch.zeros(768, device=device)
    _native.stats_fold(tot_sq, sq, tot_f, fs)
    assert rel(tot_sq, (x.double() ** 2).sum(0)) <= STATS_TOL
    assert rel(tot_f, x.double().sum(0)) <= 1e-5


def _finish_pair(device, kind, d, count, first, seed):
    g = torch.Generator().manual_seed(seed)
    sum_sq = (torch.rand(d, generator=g) * 10 + 0.1) * count
    sum_first = torch.randn(d, generator=g) * count
    prev_ema = torch.rand(d, generator=g) + 0.5
    prev_mean = torch.randn(d, generator=g) * 0.3
    # oracle
    st = {"a_sum": sum_sq.clone(), "a_count": count, "a_first_sum": sum_first.clone()}
    if not first:
        st["a_ema"] = prev_ema.clone()
        st["a_mean_ema"] = prev_mean.clone()
    if kind == 2:
        sb = {"b_sum": sum_sq.clone(), "b_count": count}
        if not first:
            sb["b_ema"] = prev_ema.clone()
        inv_ref = O.finish_b(sb, count)
        ref = dict(ema=sb["b_ema"], inv=inv_ref)
    else:
        fac, _ = O.finish_a(st, rank_one=(kind == 1))
        ref = dict(ema=st["a_ema"])
        if kind == 1:
            ref.update(mean_ema=st["a_mean_ema"], inv=fac[0], z=fac[1], kappa=fac[2])
        else:
            ref.update(inv=fac)
    # gpu (slots carry part of the sum to exercise the fold)
    t = lambda v: v.clone().to(device)
    s_sq = t(sum_sq * 0.25)
    slots_sq = torch.zeros(4, d, device=device)
    slots_sq[1] = t(sum_sq * 0.75)
    ema = t(prev_ema) if not first else torch.empty(d, device=device)
    inv = torch.empty(d, device=device)
    desc = _native.FinishDesc(sum_sq=s_sq.data_ptr(), slots_sq=slots_sq.data_ptr(), ema=ema.data_ptr(),
                              inv=inv.data_ptr(), n=d, count=count, n_slots=4, kind=kind, first=int(first))
    out = dict(ema=ema, inv=inv)
    keep = []
    if kind == 1:
        s_f = t(sum_first * 0.5)
        slots_f = torch.zeros(4, d, device=device)
        slots_f[3] = t(sum_first * 0.5)
        mean_ema = t(prev_mean) if not first else torch.empty(d, device=device)
        z = torch.empty(d, device=device)
        kappa = torch.empty(1, device=device)
        desc.sum_first, desc.slots_first, desc.mean_ema = s_f.data_ptr(), slots_f.data_ptr(), mean_ema.data_ptr()
        desc.z, desc.kappa = z.data_ptr(), kappa.data_ptr()
        out.update(mean_ema=mean_ema, z=z, kappa=kappa)
        keep += [s_f, slots_f]
    _native.stats_finish([desc], 0.97, device)
    torch.cuda.synchronize()
    assert torch.count_nonzero(s_sq) == 0 and torch.count_nonzero(slots_sq) == 0
    return out, ref


@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("first", [True, False])
@pytest.mark.parametrize("d", [4, 768, 3072])
def test_finish_matches_oracle(device, kind, first, d):
    out, ref = _finish_pair(device, kind, d, count=16384 * 8, first=first, seed=kind * 10 + d)
    assert rel(out["ema"], ref["ema"]) <= STATS_TOL
    if kind == 1:
        assert rel(out["mean_ema"], ref["mean_ema"]) <= STATS_TOL
        assert rel(out["z"], ref["z"]) <= 1e-5
        assert abs(out["kappa"].item() - float(ref["kappa"])) <= 1e-5 * abs(float(ref["kappa"]))
    assert rel(out["inv"], ref["inv"]) <= 1e-5
