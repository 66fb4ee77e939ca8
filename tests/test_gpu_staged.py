"""The staged finish and AdamW entry points (one launch for a whole
descriptor table in device memory, written on the stream through the kernel
arguments of 3840-byte upload launches) against
the by-value calls (one launch per 32 finish / 56 AdamW descriptors):
bit-identical results, on tables longer than one by-value launch takes and
on consecutive calls that cycle the staging ring with tables of different
sizes."""
import pytest
import torch

from sandmuon_amd import _native

pytestmark = pytest.mark.gpu


def _finish_case(device, n_desc, seed):
    """n_desc finish descriptors over fresh tensors: kinds 0, 1, 2 in turn,
    vector lengths 4 to 3072, some first steps; returns (descs, tensors)."""
    g = torch.Generator().manual_seed(seed)
    lens = [4, 96, 768, 1000, 3072]
    descs, keep = [], []
    for i in range(n_desc):
        kind, d = i % 3, lens[i % len(lens)]
        first = i % 4 == 0
        t = lambda *shape: (torch.rand(*shape, generator=g) + 0.1).to(device)
        s_sq, slots_sq = t(d), t(3, d)
        ema, inv = t(d), torch.zeros(d, device=device)
        desc = _native.FinishDesc(sum_sq=s_sq.data_ptr(), slots_sq=slots_sq.data_ptr(), ema=ema.data_ptr(),
                                  inv=inv.data_ptr(), n=d, count=1000 + i, n_slots=3, kind=kind, first=int(first))
        ts = dict(s_sq=s_sq, slots_sq=slots_sq, ema=ema, inv=inv)
        if kind == 1:
            s_f, slots_f = (torch.randn(d, generator=g) * 0.1).to(device), (torch.randn(3, d, generator=g) * 0.1).to(device)
            mean_ema, z, kappa = t(d) - 0.5, torch.zeros(d, device=device), torch.zeros(1, device=device)
            desc.sum_first, desc.slots_first, desc.mean_ema = s_f.data_ptr(), slots_f.data_ptr(), mean_ema.data_ptr()
            desc.z, desc.kappa = z.data_ptr(), kappa.data_ptr()
            ts.update(s_f=s_f, slots_f=slots_f, mean_ema=mean_ema, z=z, kappa=kappa)
        descs.append(desc)
        keep.append(ts)
    return descs, keep


@pytest.mark.parametrize("n_desc", [33, 90, 7])
def test_staged_finish_equals_the_batched_calls(device, n_desc):
    stage = _native.DescriptorStage(device)
    for rep in range(2):  # the second call takes the other slot of the ring
        a_descs, a = _finish_case(device, n_desc + 11 * rep, 5 + rep)
        b_descs, b = _finish_case(device, n_desc + 11 * rep, 5 + rep)
        _native.stats_finish(a_descs, 0.97, device)  # by value: one pair of launches per 32
        _native.stats_finish(b_descs, 0.97, device, stage)
        torch.cuda.synchronize()
        for ta, tb in zip(a, b):
            for key in ta:
                assert torch.equal(ta[key], tb[key]), (rep, key)
            assert torch.count_nonzero(tb["s_sq"]) == 0 and torch.count_nonzero(tb["slots_sq"]) == 0


def _adamw_case(device, n_desc, seed):
    g = torch.Generator().manual_seed(seed)
    sizes = [1, 7, 256, 1000, 4096, 70000]
    descs, keep, off = [], [], 0
    for i in range(n_desc):
        n = sizes[i % len(sizes)] + i
        pdt = [torch.float32, torch.bfloat16, torch.float16][i % 3]
        gdt = torch.float32 if i % 2 == 0 else torch.bfloat16
        p = (torch.randn(n, generator=g) * 0.02).to(pdt).to(device)
        gr = (torch.randn(n, generator=g) * 1e-3).to(gdt).to(device)
        m = (torch.randn(n, generator=g) * 1e-4).to(device)
        v = (torch.rand(n, generator=g) * 1e-6).to(device)
        step = 1 + i % 5
        descs.append(_native.AdamwDesc(param=p.data_ptr(), grad=gr.data_ptr(), exp_avg=m.data_ptr(),
                                       exp_avg_sq=v.data_ptr(), n=n, offset=off, bias1=1 - 0.9 ** step,
                                       bias2=1 - 0.95 ** step, grad_dtype=_native.dtype_code(gdt),
                                       param_dtype=_native.dtype_code(pdt)))
        keep.append((p, gr, m, v))
        off += n
    return descs, keep, off


@pytest.mark.parametrize("n_desc", [57, 130, 9])
def test_staged_adamw_equals_the_batched_calls(device, n_desc):
    stage = _native.DescriptorStage(device)
    for rep in range(2):
        a_descs, a, total = _adamw_case(device, n_desc - 2 * rep, 9 + rep)
        b_descs, b, _ = _adamw_case(device, n_desc - 2 * rep, 9 + rep)
        _native.adamw(a_descs, total, 3e-4, 0.9, 0.95, 1e-8, 0.1, device)  # one launch per 56
        _native.adamw(b_descs, total, 3e-4, 0.9, 0.95, 1e-8, 0.1, device, stage)
        torch.cuda.synchronize()
        for ta, tb in zip(a, b):
            for x, y in zip(ta, tb):
                assert torch.equal(x, y), rep


def test_staged_calls_in_flight_take_their_own_slots(device):
    # Several staged calls enqueued back to back behind a busy stream (a
    # finish and AdamW calls of two parameter groups per step, three steps),
    # so that none has run when the next is staged: each in-flight call keeps
    # its own device table, and every result equals the by-value calls'.
    stage = _native.DescriptorStage(device)
    cases = []
    for rep in range(3):
        fa, a = _finish_case(device, 40 + rep, 20 + rep)
        fb, b = _finish_case(device, 40 + rep, 20 + rep)
        wa, wta, tot = _adamw_case(device, 60 + rep, 30 + rep)
        wb, wtb, _ = _adamw_case(device, 60 + rep, 30 + rep)
        cases.append((fa, fb, a, b, wa, wb, wta, wtb, tot))
    torch.cuda.synchronize()
    torch.cuda._sleep(100_000_000)  # a bounded spin (tens of ms) ahead of the calls
    for fa, fb, a, b, wa, wb, wta, wtb, tot in cases:
        _native.stats_finish(fa, 0.97, device)
        _native.adamw(wa, tot, 1e-3, 0.9, 0.95, 1e-8, 0.1, device)
        _native.stats_finish(fb, 0.97, device, stage)
        _native.adamw(wb, tot, 1e-3, 0.9, 0.95, 1e-8, 0.1, device, stage)
    # every staged call is still in flight, each in a slot of its own
    assert sum(1 for sl in stage.slots if sl[1] is not None and not sl[1].query()) == 6
    torch.cuda.synchronize()
    for fa, fb, a, b, wa, wb, wta, wtb, tot in cases:
        for ta, tb in zip(a, b):
            for key in ta:
                assert torch.equal(ta[key], tb[key]), key
        for ta, tb in zip(wta, wtb):
            for x, y in zip(ta, tb):
                assert torch.equal(x, y)


@pytest.mark.gpu
def test_descriptor_stage_allocates_once_for_tables_that_fit(device):
    # All slots are allocated at the first staged call, at one size (a
    # power of two of at least 64 KiB); later calls whose tables fit take
    # those slots and allocate nothing; a larger table replaces all slots by
    # larger ones once.
    stage = _native.DescriptorStage(device)
    slot = stage.take(10_000)
    stage.done(slot)
    assert len(stage.slots) == stage.MAX_SLOTS and stage.size == 1 << 16
    tables = {sl[0].data_ptr() for sl in stage.slots}
    for n in (100, 30_000, 1 << 16, 5000) * 5:
        slot = stage.take(n)
        stage.done(slot)
    assert {sl[0].data_ptr() for sl in stage.slots} == tables
    slot = stage.take((1 << 16) + 1)
    stage.done(slot)
    assert stage.size == 1 << 17 and len(stage.slots) == stage.MAX_SLOTS
    assert all(sl[0].numel() == 1 << 17 for sl in stage.slots)
    torch.cuda.synchronize()
