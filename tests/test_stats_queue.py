"""Host logic of the hook queue (DiagonalWeightedPE._enqueue_stats /
_flush_stats), on CPU tensors with the native launches replaced by
recorders: when the queue launches, what one launch holds, and the loud
failure when a queued input changed in place.  The kernels themselves, and
bit-identity with one launch per hook call, are checked on the GPU
(tests/test_gpu_stats_batch.py)."""
import pytest
import torch

from sandmuon_amd import DiagonalWeightedPE, _native
from sandmuon_amd.optimizer import _StatsQueue


class Recorder:
    def __init__(self):
        self.batches = []   # list of [(rows data_ptr, slots data_ptr)], per launch
        self.single = []
        self.stream = 1
        self.busy = False   # what the stream query answers at a phase's first hook call

    def install(self, monkeypatch):
        monkeypatch.setattr(_native, "stats_accumulate_batch",
                            lambda entries, stream: self.batches.append(
                                [(r.data_ptr(), s.data_ptr(), stream) for r, s, _ in entries]))
        monkeypatch.setattr(_native, "stats_accumulate",
                            lambda rows, sq, fs: self.single.append((rows.data_ptr(), sq.data_ptr())))
        monkeypatch.setattr(_native, "stream_of", lambda device: self.stream)
        self.queries = 0

        def busy(device):
            self.queries += 1
            return self.busy
        monkeypatch.setattr(_native, "stream_busy", busy)
        self.waits = []
        monkeypatch.setattr(_native, "stream_wait", lambda waiter, signaler, device: self.waits.append((waiter, signaler)))
        monkeypatch.setattr(_native, "stats_slot_rows", lambda rows, n: min(n, max(1, -(-rows // 512))) if rows else 0)


def bare_optimizer(limit):
    """The queue state of an optimizer, without a model or the GPU library."""
    opt = object.__new__(DiagonalWeightedPE)
    opt._queue = _StatsQueue(limit)
    opt._slot_rows = {}
    return opt


def rows(n, d=8):
    return torch.zeros(n, d)


def test_queue_launches_once_it_holds_the_limit(monkeypatch):
    rec = Recorder()
    rec.install(monkeypatch)
    opt = bare_optimizer(limit=3 * 100 * 8 * 4)   # three 100 x 8 fp32 inputs
    slots = [torch.zeros(4, 8) for _ in range(4)]
    xs = [rows(100) for _ in range(4)]
    for x, s in zip(xs[:2], slots[:2]):
        opt._enqueue_stats(x, s, None)
    assert rec.batches == [] and len(opt._queue.entries) == 2
    opt._enqueue_stats(xs[2], slots[2], None)          # reaches the limit: one launch of all three
    assert [[p for p, _, _ in b] for b in rec.batches] == [[x.data_ptr() for x in xs[:3]]]
    assert opt._queue.entries == [] and opt._queue.nbytes == 0
    opt._enqueue_stats(xs[3], slots[3], None)
    opt._flush_stats()                                   # step(), state_dict() and close() call this
    assert [[p for p, _, _ in b] for b in rec.batches][1] == [xs[3].data_ptr()]
    opt._flush_stats()                                   # an empty queue launches nothing
    assert len(rec.batches) == 2


def test_launch_threshold_ramps_up_and_restarts(monkeypatch):
    rec = Recorder()
    rec.install(monkeypatch)
    opt = object.__new__(DiagonalWeightedPE)
    opt._queue = _StatsQueue(4000, first=800, growth=2.0)   # thresholds 800, 1600, 3200, 4000, 4000
    opt._slot_rows = {}
    x_bytes = 25 * 8 * 4                                     # 800 bytes per input
    sizes = []
    for k in range(17):                                      # 13600 bytes: exactly five launches
        opt._enqueue_stats(rows(25), torch.zeros(4, 8), None)
        if len(rec.batches) > len(sizes):
            sizes.append(len(rec.batches[-1]) * x_bytes)
    assert sizes == [800, 1600, 3200, 4000, 4000][:len(sizes)] and len(sizes) == 5
    assert opt._queue.threshold == 4000
    opt._flush_stats()
    opt._queue.restart()                                     # what step() does after its flush
    assert opt._queue.threshold == 800
    assert _StatsQueue(100).threshold == 100                 # a limit below the first batch is the threshold
    assert rec.queries == 1                                  # one stream query per phase of hooks


def test_no_ramp_when_the_stream_is_busy_at_the_first_hook_call(monkeypatch):
    rec = Recorder()
    rec.install(monkeypatch)
    rec.busy = True                                          # e.g. the step's kernels still running
    opt = object.__new__(DiagonalWeightedPE)
    opt._queue = _StatsQueue(4000, first=800, growth=2.0)
    opt._slot_rows = {}
    for k in range(10):                                      # 8000 bytes: two launches of the limit
        opt._enqueue_stats(rows(25), torch.zeros(4, 8), None)
    assert [len(b) for b in rec.batches] == [5, 5] and rec.queries == 1
    opt._flush_stats()
    opt._queue.restart()                                     # the next phase asks again
    rec.busy = False
    for k in range(2):
        opt._enqueue_stats(rows(25), torch.zeros(4, 8), None)
    # idle: the first launch takes 800 bytes, the next threshold is 1600
    assert [len(b) for b in rec.batches] == [5, 5, 1] and len(opt._queue.entries) == 1
    assert rec.queries == 2 and opt._queue.threshold == 1600


def test_same_slot_rows_or_another_stream_launch_the_queue_first(monkeypatch):
    rec = Recorder()
    rec.install(monkeypatch)
    opt = bare_optimizer(limit=1 << 30)
    sa, sb = torch.zeros(4, 8), torch.zeros(4, 8)
    x1, x2, x3, x4 = rows(10), rows(10), rows(10), rows(10)
    opt._enqueue_stats(x1, sa, None)
    opt._enqueue_stats(x2, sb, None)
    opt._enqueue_stats(x3, sa, None)                     # sa already queued: launch x1, x2 first
    assert [[p for p, _, _ in b] for b in rec.batches] == [[x1.data_ptr(), x2.data_ptr()]]
    rec.stream = 2
    opt._enqueue_stats(x4, sb, None)                     # another stream: launch x3 on its own stream,
    assert [p for p, _, _ in rec.batches[1]] == [x3.data_ptr()] and rec.batches[1][0][2] == 1
    assert rec.waits == [(2, 1)]                         # and make the current stream wait for it
    opt._flush_stats()
    assert rec.batches[2] == [(x4.data_ptr(), sb.data_ptr(), 2)]


def test_in_place_change_raises_and_empties_the_queue(monkeypatch):
    rec = Recorder()
    rec.install(monkeypatch)
    opt = bare_optimizer(limit=1 << 30)
    x = rows(10)
    opt._enqueue_stats(x, torch.zeros(4, 8), None)
    x.add_(1)
    with pytest.raises(RuntimeError, match="modified in place"):
        opt._flush_stats()
    assert rec.batches == [] and opt._queue.entries == []


def test_queue_off_and_empty_inputs(monkeypatch):
    rec = Recorder()
    rec.install(monkeypatch)
    opt = bare_optimizer(limit=0)                        # hook_batch_bytes=0: launch in the hook
    s = torch.zeros(4, 8)
    opt._enqueue_stats(rows(10), s, None)
    assert len(rec.single) == 1 and rec.batches == []
    opt = bare_optimizer(limit=1 << 30)
    opt._enqueue_stats(rows(0), s, None)                 # an empty microbatch queues nothing
    assert opt._queue.entries == []


def test_folds_read_only_the_slot_rows_calls_touched(monkeypatch):
    rec = Recorder()
    rec.install(monkeypatch)
    opt = bare_optimizer(limit=1 << 30)
    s = torch.zeros(128, 8)
    opt._enqueue_stats(rows(600), s, None)               # 2 chunks of >= 512 rows
    opt._enqueue_stats(rows(100), torch.zeros(128, 8), None)
    opt._enqueue_stats(rows(1500), torch.zeros(128, 8), None)
    assert opt._slot_rows[s.data_ptr()] == 2
    assert opt._take_slot_rows(s) == 2 and opt._take_slot_rows(s) == 1  # restarts after the fold


def test_constructor_rejects_a_negative_limit():
    with pytest.raises(ValueError, match="hook_batch_bytes"):
        DiagonalWeightedPE(torch.nn.Sequential(torch.nn.Linear(4, 4)), 1e-2, hook_batch_bytes=-1)
