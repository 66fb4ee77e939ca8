"""GPU tests of the batched statistics launch and the optimizer's hook queue.

Bar: bit-identical.  One launch over several hook inputs
(smx_stats_accumulate_batch) must add exactly what one launch per input adds,
and an optimizer whose hooks queue their inputs must end every step with the
same bits as one that launches inside each hook (hook_batch_bytes=0), which
is the path the oracle parity suites check against sandmuon/optimizer.py.
"""
import copy

import pytest
import torch
from torch import nn

from sandmuon_amd import DiagonalWeightedPE, RankOneAWeightedPE, _native
from sandmuon_amd.workloads import GPT, GPTConfig, stats_cfg3_tensor, transformer_filter

pytestmark = pytest.mark.gpu

# (rows, cols, dtype, column offset into a wider tensor): every element form
# of the kernel -- 16-byte vectors for f32/bf16/f16, the scalar forms for odd
# widths and misaligned rows -- plus fewer rows than slot rows and no rows.
SPECS = [
    (16384, 768, torch.float32, 0),
    (4096, 3072, torch.bfloat16, 0),
    (3000, 256, torch.float16, 0),
    (777, 37, torch.float32, 0),
    (500, 100, torch.bfloat16, 3),
    (90, 24, torch.float16, 1),
    (50, 8, torch.float32, 0),
    (0, 64, torch.bfloat16, 0),
    (1, 768, torch.bfloat16, 0),
]


def make_inputs(device, n):
    xs = []
    for i in range(n):
        rows, cols, dtype, off = SPECS[i % len(SPECS)]
        full = stats_cfg3_tensor(100 + i, rows, cols + off, dtype=dtype).to(device)
        xs.append(full[:, off:off + cols])
    return xs


@pytest.mark.parametrize("first", [False, True])
@pytest.mark.parametrize("n", [1, 9, 30])  # 30 inputs: more than one launch's job table
def test_batched_launch_equals_single_launches(device, first, n):
    xs = make_inputs(device, n)

    def slots(x):
        sq = torch.rand(128, x.shape[1], device=device)  # accumulate onto non-zero slots
        return sq, (torch.rand_like(sq) if first else None)

    single = [slots(x) for x in xs]
    batch = [(sq.clone(), None if fs is None else fs.clone()) for sq, fs in single]
    for x, (sq, fs) in zip(xs, single):
        _native.stats_accumulate(x, sq, fs)
    _native.stats_accumulate_batch([(x, sq, fs) for x, (sq, fs) in zip(xs, batch)], _native.stream_of(device))
    torch.cuda.synchronize()
    for i, ((s1, f1), (s2, f2)) in enumerate(zip(single, batch)):
        assert torch.equal(s1, s2), (i, SPECS[i % len(SPECS)])
        if first:
            assert torch.equal(f1, f2), (i, SPECS[i % len(SPECS)])


def test_batched_launch_rejects_shared_slot_rows(device):
    x = torch.randn(64, 32, device=device)
    sq = torch.zeros(128, 32, device=device)
    with pytest.raises(ValueError, match="overlap"):
        _native.stats_accumulate_batch([(x, sq, None), (x, sq, None)], _native.stream_of(device))


CFG = GPTConfig(vocab=211, ctx=64, layers=2, width=64, heads=4, mlp=256)


def run_steps(device, opt_cls, batch_bytes, steps=2, micro=3, stream=None, autocast=True):
    torch.manual_seed(0)
    model = GPT(CFG)
    model.init_weights(7)
    model = model.to(device)
    opt = opt_cls(model, 1e-2, module_filter=transformer_filter, hook_batch_bytes=batch_bytes)
    g = torch.Generator(device=device).manual_seed(11)
    for _ in range(steps):
        opt.zero_grad(set_to_none=True)
        for _ in range(micro):
            idx = torch.randint(0, CFG.vocab, (4, CFG.ctx), generator=g, device=device)
            s = stream or torch.cuda.current_stream(device)
            if stream is not None:
                stream.wait_stream(torch.cuda.current_stream(device))
            with torch.cuda.stream(s), torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
                loss = model(idx, idx) / micro
            with torch.cuda.stream(s):
                loss.backward()
            if stream is not None:
                torch.cuda.current_stream(device).wait_stream(stream)
        opt.step()
    torch.cuda.synchronize()
    return model, opt


def assert_same(m1, o1, m2, o2):
    for (n1, p1), (n2, p2) in zip(m1.named_parameters(), m2.named_parameters()):
        assert torch.equal(p1, p2), n1
    for p1, p2 in zip(m1.parameters(), m2.parameters()):
        s1, s2 = o1.state.get(p1, {}), o2.state.get(p2, {})
        assert s1.keys() == s2.keys()
        for k in s1:
            if torch.is_tensor(s1[k]):
                assert torch.equal(s1[k], s2[k]), k
            else:
                assert s1[k] == s2[k], k


@pytest.mark.parametrize("opt_cls", [RankOneAWeightedPE, DiagonalWeightedPE])
@pytest.mark.parametrize("batch_bytes", [None, 200_000])  # default: one launch per step; small: many, with slot conflicts
def test_queued_hooks_equal_immediate_hooks(device, opt_cls, batch_bytes):
    ref = run_steps(device, opt_cls, 0)
    got = run_steps(device, opt_cls, batch_bytes)
    assert_same(*ref, *got)


def test_queue_flushes_before_state_dict(device):
    model, opt = run_steps(device, RankOneAWeightedPE, 0, steps=1)
    ref = copy.deepcopy(opt.state_dict())
    model2, opt2 = run_steps(device, RankOneAWeightedPE, None, steps=1)
    # one more microbatch, not stepped: its statistics are queued
    for m, o in ((model, opt), (model2, opt2)):
        idx = torch.arange(4 * CFG.ctx, device=device).view(4, CFG.ctx) % CFG.vocab
        with torch.autocast("cuda", dtype=torch.bfloat16):
            m(idx, idx).backward()
    assert opt2._queue.entries, "the default limit keeps a small model's hook inputs queued"
    sd1, sd2 = opt.state_dict(), opt2.state_dict()
    assert not opt2._queue.entries
    for k, v in sd1["state"].items():
        for name, t in v.items():
            if torch.is_tensor(t):
                assert torch.equal(t, sd2["state"][k][name]), (k, name)
            else:
                assert t == sd2["state"][k][name]
    del ref


def test_hooks_on_a_side_stream(device):
    ref = run_steps(device, RankOneAWeightedPE, 0)
    side = torch.cuda.Stream(device)  # default priority
    got = run_steps(device, RankOneAWeightedPE, None, stream=side)
    assert_same(*ref, *got)


def test_in_place_change_of_a_queued_input_raises(device):
    torch.manual_seed(0)
    model = nn.Sequential(nn.Linear(32, 32), nn.Linear(32, 8)).to(device)
    opt = DiagonalWeightedPE(model, 1e-2)
    x = torch.randn(16, 32, device=device)
    model(x).sum().backward()
    assert opt._queue.entries
    x.mul_(2)  # after the forward hook queued x
    with pytest.raises(RuntimeError, match="modified in place"):
        opt.step()
    assert not opt._queue.entries


def test_hook_input_from_another_stream_is_kept_until_its_launch(device):
    """A hook input allocated on another stream and dropped right after its
    hook.  The queued launch runs later, on the hook's stream (kept busy
    here by a bounded sleep kernel); the allocator must not hand the input's
    memory to a new allocation on its own stream before then, so the launch
    records its use of every input on its stream."""
    torch.manual_seed(5)
    model = nn.Sequential(nn.Linear(256, 64)).to(device)
    opt = DiagonalWeightedPE(model, 1e-2)
    p = model[0].weight
    side = torch.cuda.Stream(device)  # default priority
    cur = torch.cuda.current_stream(device)
    rows, cols = 8192, 256
    with torch.cuda.stream(side):
        x = torch.randn(rows, cols, device=device)
    cur.wait_stream(side)
    want = x.double().square().sum(0)
    torch.cuda._sleep(50_000_000)
    opt._accumulate_a(p, x)
    opt._flush_stats()
    del x
    with torch.cuda.stream(side):
        junk = torch.full((rows, cols), 1e3, device=device)
    torch.cuda.synchronize()
    _, sq, _ = opt._slots[(id(p), "a")]
    got = sq.double().sum(0)
    assert ((got - want).norm() / want.norm()).item() <= 1e-6
    del junk
    opt.close()


def test_queue_launched_on_the_hook_stream_orders_the_current_stream(device):
    """Hooks run on a side stream (kept busy by a bounded sleep kernel); the
    queue is launched from the default stream, on the hooks' stream, and the
    default stream must wait for that launch before it reads the slot rows."""
    torch.manual_seed(6)
    model = nn.Sequential(nn.Linear(256, 64)).to(device)
    opt = DiagonalWeightedPE(model, 1e-2)
    p = model[0].weight
    x = torch.randn(8192, 256, device=device)
    want = x.double().square().sum(0)
    side = torch.cuda.Stream(device)  # default priority
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        torch.cuda._sleep(50_000_000)
        opt._accumulate_a(p, x)
    x.record_stream(side)
    opt._flush_stats()  # from the default stream
    _, sq, _ = opt._slots[(id(p), "a")]
    got = sq.double().sum(0)  # enqueued on the default stream
    torch.cuda.synchronize()
    assert ((got - want).norm() / want.norm()).item() <= 1e-6
    opt.close()


def test_ramp_only_when_the_hook_stream_is_idle(device):
    """The first hook call of a phase asks whether its stream still has work:
    busy (here a bounded sleep kernel) -> every launch takes the full batch
    size; idle -> the threshold ramps from the first size.  A stream under
    graph capture counts as busy and is not queried."""
    model = nn.Sequential(nn.Linear(256, 64)).to(device)
    opt = DiagonalWeightedPE(model, 1e-2, hook_batch_bytes=64 << 20)
    q = opt._queue
    q.first = 1 << 20
    p = model[0].weight
    x = torch.randn(64, 256, device=device)           # 64 KB: stays queued
    opt._accumulate_a(p, x)                           # allocates the slot rows (a fill kernel)
    opt._flush_stats()
    torch.cuda.synchronize()
    q.restart()
    opt._accumulate_a(p, x)                           # idle stream: ramp
    assert q.threshold == 1 << 20 and not q.fresh
    opt._flush_stats()
    q.restart()
    torch.cuda._sleep(50_000_000)
    opt._accumulate_a(p, x)                           # busy stream: full size
    assert q.threshold == 64 << 20
    opt._flush_stats()
    torch.cuda.synchronize()

    g = torch.cuda.CUDAGraph()
    y = torch.zeros(4, device=device)
    s = torch.cuda.Stream(device)
    s.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(s):
        y.add_(1)                                     # warm-up of the captured op
    torch.cuda.current_stream(device).wait_stream(s)
    with torch.cuda.graph(g):
        busy = _native.stream_busy(y.device)
        y.add_(1)
    assert busy
    g.replay()
    torch.cuda.synchronize()
    assert y.tolist() == [2.0] * 4
    opt.close()
