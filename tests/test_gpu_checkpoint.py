"""state_dict() / load_state_dict() of the GPU build (sandmuon/optimizer.py:
96-321, torch.optim.Optimizer's, with the state kept float32 on load).

* The saved structure (param groups, state keys, dtypes, shapes, int counts
  and int AdamW step) equals the reference's, recorded by the reference in
  tests/golden/state_dict.json.
* Resuming from a checkpoint is bit-identical to an uninterrupted run (the
  build-vs-build pattern of the reference's tests/test_optimizer.py:95-113).
* Hook statistics still pending in the slot buffers are folded into the
  saved a_sum / b_sum (checked against an FP64 brute force), and loading a
  checkpoint discards pending partials.
* With bf16 parameters the loaded statistics, EMA, momentum and moment
  tensors stay float32 (torch would cast them to bf16) and a resumed run
  is bit-identical to an uninterrupted one.
* A checkpoint whose AdamW `step` is a tensor (the historical trainer's
  format, reproduction/odl/optim/diagonal_weighted_pe.py:487-493) loads and
  continues exactly like the int form.
"""
import copy
import json
from pathlib import Path

import pytest
import torch

from sandmuon_amd import RankOneAWeightedPE
from sandmuon_amd.workloads import GPT, GPT_TINY, transformer_filter

pytestmark = pytest.mark.gpu

FIXTURE = Path(__file__).resolve().parent / "golden" / "state_dict.json"


def batches(device, seed, n=2):
    g = torch.Generator(device="cpu").manual_seed(seed)
    out = []
    for _ in range(n):
        idx = torch.randint(0, GPT_TINY.vocab, (3, GPT_TINY.ctx), generator=g)
        tgt = torch.randint(0, GPT_TINY.vocab, (3, GPT_TINY.ctx), generator=g)
        out.append((idx.to(device), tgt.to(device)))
    return out


def fresh(device, seed=11):
    model = GPT(GPT_TINY)
    model.init_weights(seed)
    return model.to(device)


def backward(model, data):
    for idx, tgt in data:
        (model(idx, tgt) / len(data)).backward()


def train_step(model, opt, data):
    backward(model, data)
    opt.step()
    opt.zero_grad(set_to_none=True)


def cpu_copy(sd):
    return copy.deepcopy({"state": {k: {n: (v.detach().cpu().clone() if torch.is_tensor(v) else v)
                                          for n, v in s.items()} for k, s in sd["state"].items()},
                          "param_groups": sd["param_groups"]})


def params_of(model):
    return {n: p.detach().clone() for n, p in model.named_parameters()}


def record(device, params, names, data, dtype=torch.float32):
    """Hook inputs, output cotangents and gradients of one effective batch,
    computed once on a separate copy of the model at `params` (in `dtype`),
    so that two optimizers can be fed bit-identical inputs (the model's own
    backward is not bit-reproducible: the embedding backward uses atomics)."""
    model = fresh(device).to(dtype)
    with torch.no_grad():
        for n, p in model.named_parameters():
            p.copy_(params[n])
    recs, handles = [], []
    modules = dict(model.named_modules())
    for name in names:
        def hook(module, inputs, output, key=name):
            recs.append((key, "a", inputs[0].detach().clone()))

            def th(grad):
                recs.append((key, "b", grad.detach().clone()))
                return grad
            output.register_hook(th)
        handles.append(modules[name[: -len(".weight")]].register_forward_hook(hook))
    backward(model, data)
    for h in handles:
        h.remove()
    return recs, {n: p.grad.detach().clone() for n, p in model.named_parameters()}


def replay_step(model, opt, recs, grads):
    """One optimizer step from recorded inputs, through the hook bodies."""
    named = dict(model.named_parameters())
    for key, side, t in recs:
        p = named[key]
        if side == "b":
            opt._accumulate_b(p, t)
        elif opt.a_sources[id(p)] is p:
            opt._accumulate_a(p, t)
    for n, p in named.items():
        p.grad = grads[n].clone()
    opt.step()
    opt.zero_grad(set_to_none=True)


def test_state_dict_structure_matches_reference(device):
    model = fresh(device)
    opt = RankOneAWeightedPE(model, lr=3e-3, module_filter=transformer_filter)
    train_step(model, opt, batches(device, 1))
    sd = opt.state_dict()
    ref = json.loads(FIXTURE.read_text())
    assert len(sd["param_groups"]) == len(ref["param_groups"])
    for got, want in zip(sd["param_groups"], ref["param_groups"]):
        assert set(got) == set(want)
        for key, value in want.items():
            if key == "params":
                assert len(got["params"]) == value
            elif isinstance(value, list):
                assert list(got[key]) == value, key
            else:
                assert got[key] == value, key
    assert {str(k) for k in sd["state"]} == set(ref["state"])
    for k, entry in sd["state"].items():
        want = ref["state"][str(k)]
        assert set(entry) == set(want), k
        for name, spec in want.items():
            value = entry[name]
            if "type" in spec:
                assert type(value).__name__ == spec["type"], (k, name)
            else:
                assert torch.is_tensor(value) and str(value.dtype) == spec["dtype"], (k, name)
                assert list(value.shape) == spec["tensor"], (k, name)
    opt.close()


def test_resume_is_bit_identical(device):
    model_a = fresh(device)
    opt_a = RankOneAWeightedPE(model_a, lr=3e-3, module_filter=transformer_filter)
    names = list(opt_a.named_matrices)
    replay_step(model_a, opt_a, *record(device, params_of(model_a), names, batches(device, 2)))
    saved = cpu_copy(opt_a.state_dict())
    saved_params = params_of(model_a)
    step2 = record(device, saved_params, names, batches(device, 3))
    replay_step(model_a, opt_a, *step2)

    model_b = fresh(device, seed=99)  # every value is overwritten below
    with torch.no_grad():
        for n, p in model_b.named_parameters():
            p.copy_(saved_params[n])
    opt_b = RankOneAWeightedPE(model_b, lr=3e-3, module_filter=transformer_filter)
    opt_b.load_state_dict(saved)
    replay_step(model_b, opt_b, *step2)
    for (n, pa), (_, pb) in zip(model_a.named_parameters(), model_b.named_parameters()):
        assert torch.equal(pa, pb), n
    for pa, pb in zip(opt_a.state.values(), opt_b.state.values()):
        assert set(pa) == set(pb)
        for key in pa:
            if torch.is_tensor(pa[key]):
                assert torch.equal(pa[key], pb[key]), key
            else:
                assert pa[key] == pb[key], key
    opt_a.close()
    opt_b.close()


def test_pending_statistics_are_saved_and_pending_partials_dropped_on_load(device):
    model = fresh(device)
    opt = RankOneAWeightedPE(model, lr=3e-3, module_filter=transformer_filter)
    train_step(model, opt, batches(device, 4))
    # Hooks fire, no step: the partial sums sit in the slot buffers.
    captured = {}
    name_of = {id(p): n for n, p in opt.named_matrices.items()}
    handles = []
    for name, mod in model.named_modules():
        w = getattr(mod, "weight", None)
        if w is not None and id(w) in name_of:
            def hook(module, inputs, output, key=name_of[id(w)]):
                captured.setdefault(key, []).append(inputs[0].detach().double().reshape(-1, inputs[0].shape[-1]))
            handles.append(mod.register_forward_hook(hook))
    backward(model, batches(device, 5))
    for h in handles:
        h.remove()
    sd = opt.state_dict()
    for key, xs in captured.items():
        p = opt.named_matrices[key]
        if opt.a_sources[id(p)] is not p:
            continue
        index = next(i for i, q in enumerate(opt.param_groups[0]["params"]) if q is p)
        want = sum((x * x).sum(0) for x in xs)
        got = sd["state"][index]["a_sum"].double()
        assert ((got - want).norm() / want.norm()).item() <= 1e-6, key
    # Loading a checkpoint discards the partials of hooks that ran since.
    saved = cpu_copy(sd)
    backward(model, batches(device, 6))
    opt.zero_grad(set_to_none=True)
    opt.load_state_dict(saved)
    again = opt.state_dict()
    for k, entry in saved["state"].items():
        for name, value in entry.items():
            if torch.is_tensor(value):
                assert torch.equal(again["state"][k][name].cpu(), value), (k, name)
    opt.close()


def test_tensor_adamw_step_loads_like_int(device):
    model = fresh(device)
    opt = RankOneAWeightedPE(model, lr=3e-3, module_filter=transformer_filter)
    names = list(opt.named_matrices)
    replay_step(model, opt, *record(device, params_of(model), names, batches(device, 7)))
    saved = cpu_copy(opt.state_dict())
    start = params_of(model)
    step2 = record(device, start, names, batches(device, 8))
    tensor_form = copy.deepcopy(saved)
    n_aux = 0
    for entry in tensor_form["state"].values():
        if "step" in entry:
            entry["step"] = torch.tensor(float(entry["step"]))
            n_aux += 1
    assert n_aux > 0
    results = []
    for ckpt in (saved, tensor_form):
        m = fresh(device, seed=99)
        with torch.no_grad():
            for n, p in m.named_parameters():
                p.copy_(start[n])
        o = RankOneAWeightedPE(m, lr=3e-3, module_filter=transformer_filter)
        o.load_state_dict(copy.deepcopy(ckpt))
        replay_step(m, o, *step2)
        results.append(params_of(m))
        steps = [s["step"] for s in o.state.values() if "step" in s]
        assert steps and all(isinstance(s, int) and s == 2 for s in steps)
        o.close()
    for n in results[0]:
        assert torch.equal(results[0][n], results[1][n]), n
    opt.close()


def test_bf16_parameters_resume_with_float32_state(device):
    """torch's load_state_dict casts floating state to the parameter dtype;
    the build keeps every statistic, EMA, momentum and moment float32 (the
    kernels read and write FP32), restored from the saved values.  With bf16
    parameters a resumed run is bit-identical to an uninterrupted one."""
    def bf16_model(seed=11):
        return fresh(device, seed).to(torch.bfloat16)

    model_a = bf16_model()
    opt_a = RankOneAWeightedPE(model_a, lr=3e-3, module_filter=transformer_filter)
    names = list(opt_a.named_matrices)
    replay_step(model_a, opt_a, *record(device, params_of(model_a), names, batches(device, 12), torch.bfloat16))
    saved = cpu_copy(opt_a.state_dict())
    float_keys = set()
    for entry in saved["state"].values():
        for key, value in entry.items():
            if torch.is_tensor(value):
                assert value.dtype == torch.float32, key
                float_keys.add(key)
    assert {"a_sum", "a_first_sum", "b_sum", "a_ema", "a_mean_ema", "b_ema", "momentum_buffer",
            "exp_avg", "exp_avg_sq"} <= float_keys
    saved_params = params_of(model_a)
    step2 = record(device, saved_params, names, batches(device, 13), torch.bfloat16)
    replay_step(model_a, opt_a, *step2)

    model_b = bf16_model(seed=99)
    with torch.no_grad():
        for n, p in model_b.named_parameters():
            p.copy_(saved_params[n])
    opt_b = RankOneAWeightedPE(model_b, lr=3e-3, module_filter=transformer_filter)
    opt_b.load_state_dict(saved)
    for k, entry in opt_b.state_dict()["state"].items():
        for key, value in entry.items():
            if torch.is_tensor(value):
                assert value.dtype == torch.float32 and value.is_contiguous(), (k, key)
                assert torch.equal(value.cpu(), saved["state"][k][key]), (k, key)
    replay_step(model_b, opt_b, *step2)
    for (n, pa), (_, pb) in zip(model_a.named_parameters(), model_b.named_parameters()):
        assert pa.dtype == torch.bfloat16
        assert torch.equal(pa, pb), n
    for pa, pb in zip(opt_a.state.values(), opt_b.state.values()):
        for key in pa:
            if torch.is_tensor(pa[key]):
                assert pb[key].dtype == torch.float32, key
                assert torch.equal(pa[key], pb[key]), key
    opt_a.close()
    opt_b.close()

