"""The historical ODL plugin classes on the GPU (reproduction/odl/optim/
diagonal_weighted_pe.py:165-564, registry.py:57-75).

Where the historical and portable optimizers share the arithmetic (the
statistics, factors, momentum .8, whiten, S8, mapback, graft and AdamW), a
historical step must equal the portable step bit for bit on the same
inputs; the tests then pin what the historical boundary changes: the fixed
momentum, the closure without gradients, the float32 tensor AdamW step of
its checkpoints and the cotangent-count message.
"""
import copy

import pytest
import torch

from sandmuon_amd import RankOneAWeightedPE as PortableRankOne
from sandmuon_amd import odl
from sandmuon_amd.workloads import transformer_filter

from test_gpu_checkpoint import batches, cpu_copy, fresh, params_of, record, replay_step

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name,cls,rank_one", [("sand_muon", odl.DiagonalWeightedPE, False),
                                               ("muon_raw_diagonal_weighted_pe", odl.DiagonalWeightedPE, False),
                                               ("sand_muon_rank1", odl.RankOneAWeightedPE, True)])
def test_factories_build_the_historical_classes(device, name, cls, rank_one):
    model = fresh(device)
    opt = odl.create_optimizer(model, lr=2e-3, betas=(.1, .2), weight_decay=.5, optimizer_type=name)
    assert type(opt) is cls and opt.rank_one_a is rank_one
    assert opt.param_groups[0]["lr"] == 2e-3 and opt.param_groups[1]["weight_decay"] == .01
    if rank_one:
        assert opt.split_sides is False
    assert set(opt.named_matrices) == {n for n, _ in model.named_parameters()
                                       if n.startswith("transformer.h.") and n.endswith("proj.weight")
                                       or ".mlp.c_fc.weight" in n}
    opt.close()


def test_historical_step_equals_portable_step_with_fixed_momentum(device):
    model_h, model_p = fresh(device), fresh(device)
    hist = odl.RankOneAWeightedPE(model_h, 3e-3, split_sides=True)
    port = PortableRankOne(model_p, 3e-3, module_filter=transformer_filter)
    assert list(hist.named_matrices) == list(port.named_matrices)
    hist.param_groups[0]["momentum"] = .5  # ignored: the historical momentum is fixed at .8
    names = list(port.named_matrices)
    for seed in (21, 22):
        data = record(device, params_of(model_p), names, batches(device, seed))
        replay_step(model_h, hist, *data)
        replay_step(model_p, port, *data)
        for (n, a), (_, b) in zip(model_h.named_parameters(), model_p.named_parameters()):
            assert torch.equal(a, b), n
    hist.close()
    port.close()


def test_closure_runs_without_gradients(device):
    model = fresh(device)
    opt = odl.DiagonalWeightedPE(model, 3e-3)
    names = list(opt.named_matrices)
    recs, grads = record(device, params_of(model), names, batches(device, 23))
    named = dict(model.named_parameters())
    for key, side, t in recs:
        if side == "b":
            opt._accumulate_b(named[key], t)
        elif opt.a_sources[id(named[key])] is named[key]:
            opt._accumulate_a(named[key], t)
    for n, p in named.items():
        p.grad = grads[n].clone()
    seen = []

    def closure():
        seen.append(torch.is_grad_enabled())
        return torch.tensor(1.5)
    assert opt.step(closure).item() == 1.5
    assert seen == [False]
    opt.close()


def test_checkpoint_step_is_a_float32_tensor_and_resumes_bit_identically(device):
    model_a = fresh(device)
    opt_a = odl.RankOneAWeightedPE(model_a, 3e-3)
    names = list(opt_a.named_matrices)
    replay_step(model_a, opt_a, *record(device, params_of(model_a), names, batches(device, 24)))
    sd = opt_a.state_dict()
    steps = [e["step"] for e in sd["state"].values() if "step" in e]
    assert steps and all(torch.is_tensor(s) and s.dtype == torch.float32 and s.device.type == "cuda"
                         and s.item() == 1.0 for s in steps)
    # the optimizer's own state keeps the host count
    assert all(isinstance(s["step"], int) for s in opt_a.state.values() if "step" in s)
    saved, saved_params = cpu_copy(sd), params_of(model_a)
    step2 = record(device, saved_params, names, batches(device, 25))
    replay_step(model_a, opt_a, *step2)

    model_b = fresh(device, seed=99)
    with torch.no_grad():
        for n, p in model_b.named_parameters():
            p.copy_(saved_params[n])
    opt_b = odl.RankOneAWeightedPE(model_b, 3e-3)
    opt_b.load_state_dict(copy.deepcopy(saved))
    replay_step(model_b, opt_b, *step2)
    for (n, pa), (_, pb) in zip(model_a.named_parameters(), model_b.named_parameters()):
        assert torch.equal(pa, pb), n
    opt_a.close()
    opt_b.close()


def test_cotangent_mismatch_message(device):
    model = fresh(device)
    opt = odl.DiagonalWeightedPE(model, 3e-3)
    names = list(opt.named_matrices)
    recs, grads = record(device, params_of(model), names, batches(device, 26))
    named = dict(model.named_parameters())
    for key, side, t in recs:
        if side == "a" and opt.a_sources[id(named[key])] is named[key]:
            opt._accumulate_a(named[key], t)
    for n, p in named.items():
        p.grad = grads[n].clone()
    with pytest.raises(RuntimeError) as e:
        opt.step()
    assert str(e.value) == "Missing or mismatched cotangent statistics: " + names[0]
    opt.close()
