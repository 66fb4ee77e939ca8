"""End-to-end GPU parity of RankOneAWeightedPE / DiagonalWeightedPE against
the CPU oracle on identical inputs.

The GPU model runs forward/backward; every hooked activation and cotangent
and every gradient is captured and fed to the oracle, so both sides see the
same numbers.  Gates (north star): statistics/EMA state rel. error <= 1e-6;
per-matrix update direction rel. Frobenius error <= 1e-4 (fp32 mode) and
<= 1e-2 (comp_bf16 mode).  AdamW parameters: elementwise FP32 (<= 1e-6).
"""
import copy
import math

import pytest
import torch
from torch import nn

from oracle import sandmuon_oracle as O
from sandmuon_amd import DiagonalWeightedPE, RankOneAWeightedPE
from sandmuon_amd.workloads import GPT, GPT_TINY, rng, transformer_filter

pytestmark = pytest.mark.gpu

DIR_TOL = {"fp32": 1e-4, "comp_bf16": 1e-2, "mixed": 1e-2}
STATS_TOL = 1e-6


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-300)).item()


class Capture:
    """Records the inputs and output cotangents of the selected modules."""

    def __init__(self, model, names):
        self.records = []
        self.handles = []
        modules = dict(model.named_modules())
        for name in names:
            mod = modules[name[: -len(".weight")]]
            self.handles.append(mod.register_forward_hook(self._hook(name)))

    def _hook(self, name):
        def hook(module, inputs, output):
            self.records.append((name, "a", inputs[0].detach().float().cpu().clone()))

            def th(grad):
                self.records.append((name, "b", grad.detach().float().cpu().clone()))
                return grad
            output.register_hook(th)
        return hook

    def drain(self):
        out, self.records = self.records, []
        return out

    def close(self):
        for h in self.handles:
            h.remove()


class Pair:
    """A GPU model + optimizer and a CPU copy + oracle stepped in lockstep:
    the oracle is fed the GPU side's captured hook inputs and gradients."""

    def __init__(self, device, model, opt_cls, mode, lr, module_filter=None):
        self.device, self.lr = device, lr
        self.gpu_model = model.to(device)
        self.cpu_model = copy.deepcopy(model).cpu()
        self.opt = opt_cls(self.gpu_model, lr, module_filter=module_filter, s8_mode=mode)
        self.ora = O.OracleOptimizer(self.cpu_model, lr, rank_one_a=self.opt.rank_one_a,
                                     module_filter=module_filter, hooks=False)
        assert list(self.opt.named_matrices) == list(self.ora.matrices)
        self.cap = Capture(self.gpu_model, self.opt.named_matrices)

    def step(self, batches, loss_fn, prepare=None):
        """One step on both sides; `prepare(gpu_model)` may rewrite the GPU
        gradients (same values) after the backward passes."""
        opt, ora, device = self.opt, self.ora, self.device
        gparams = dict(self.gpu_model.named_parameters())
        cparams = dict(self.cpu_model.named_parameters())
        opt.zero_grad(set_to_none=True)
        for x, y in batches:
            loss_fn(self.gpu_model, x.to(device), y.to(device)).backward()
        if prepare is not None:
            prepare(self.gpu_model)
        for name, kind, t in self.cap.drain():
            ora.feed(name, x=t if kind == "a" else None, delta=t if kind == "b" else None)
        with torch.no_grad():
            for n, p in gparams.items():
                cparams[n].copy_(p.detach().cpu())
                cparams[n].grad = None if p.grad is None else p.grad.detach().cpu().clone()
        before = {n: p.detach().clone() for n, p in gparams.items()}
        opt.step()
        ora.step()
        torch.cuda.synchronize()
        entry = (before, {n: p.detach().clone() for n, p in gparams.items()},
                 {n: p.detach().clone() for n, p in cparams.items()})
        # state comparisons
        for n, p in opt.named_matrices.items():
            gs, cs = opt.state[p], ora.st(ora.matrices[n])
            for key in ("a_ema", "a_mean_ema", "b_ema"):
                if key in cs:
                    assert key in gs, (n, key)
                    assert rel(gs[key], cs[key]) <= STATS_TOL, (n, key, rel(gs[key], cs[key]))
            for key in ("a_count", "b_count"):
                if key in cs:
                    assert gs[key] == cs[key] == 0
            assert rel(gs["momentum_buffer"], cs["momentum_buffer"]) <= 1e-6
        return entry

    def close(self):
        self.cap.close()
        self.opt.close()


def run_pair(device, model, batches, loss_fn, opt_cls, mode, lr, steps, module_filter=None):
    pair = Pair(device, model, opt_cls, mode, lr, module_filter)
    history = [pair.step(batches, loss_fn) for _ in range(steps)]
    pair.close()
    return history, pair.opt, pair.ora


def check_directions(history, opt, lr, mode):
    worst = 0.0
    for before, after_g, after_c in history:
        for n in opt.named_matrices:
            dg = (before[n] - after_g[n]).double().cpu() / lr
            dc = (before[n].cpu() - after_c[n]).double() / lr
            e = rel(dg, dc)
            worst = max(worst, e)
            assert e <= DIR_TOL[mode], (n, e)
            # Frobenius graft: ||dW|| / lr = sqrt(rows) (tests/test_optimizer.py:215-237)
            assert abs(dg.norm().item() - math.sqrt(before[n].shape[0])) <= 1e-4 * math.sqrt(before[n].shape[0])
    return worst


def check_aux(history, opt, ora=None):
    # AdamW is elementwise FP32: parameters agree to a few ulp.  (The update
    # delta itself is not compared: for weights near 1 one ulp of p is
    # ~1e-4 of a 1e-3-scale step.)
    for before, after_g, after_c in history:
        for n, p in after_g.items():
            if n in opt.named_matrices:
                continue
            assert rel(after_g[n], after_c[n]) <= 1e-6, n
    if ora is not None:
        for p_g, p_c in zip(opt.param_groups[-1]["params"], ora.aux):
            gs, cs = opt.state[p_g], ora.st(p_c)
            assert gs["step"] == cs["step"] and isinstance(gs["step"], int)
            assert rel(gs["exp_avg"], cs["exp_avg"]) <= 1e-6
            assert rel(gs["exp_avg_sq"], cs["exp_avg_sq"]) <= 1e-6


def mse(model, x, y):
    return (model(x) - y).square().mean()


@pytest.mark.parametrize("mode", ["fp32", "comp_bf16", "mixed"])
def test_cfg1_single_linear_768(device, mode):
    """BASELINE cfg1: fp32 Linear 768->768, W ~ N(0, .02), bias 0, lr 1e-2,
    4 microbatches of 16x1024 tokens, x = N(0,1) + mu_c (mu_c ~ N(0, .5)),
    MSE against N(0,1) targets."""
    r = rng(1001)
    model = nn.Linear(768, 768)
    with torch.no_grad():
        model.weight.copy_(torch.from_numpy(r.normal(0, 0.02, (768, 768))).float())
        model.bias.zero_()
    mu = torch.from_numpy(r.normal(0, 0.5, 768)).float()
    batches = []
    for _ in range(4):
        x = torch.from_numpy(r.standard_normal((16, 1024, 768))).float() + mu
        y = torch.from_numpy(r.standard_normal((16, 1024, 768))).float()
        batches.append((x, y))

    class Wrap(nn.Module):
        def __init__(self, lin):
            super().__init__()
            self.proj = lin

        def forward(self, x):
            return self.proj(x)

    loss = lambda m, x, y: (m(x) - y).square().mean() / 4
    hist, opt, _ = run_pair(device, Wrap(model), batches, loss, RankOneAWeightedPE, mode, 1e-2, steps=1)
    worst = check_directions(hist, opt, 1e-2, mode)
    print(f"cfg1 {mode}: worst direction rel err {worst:.3e}")
    check_aux(hist, opt)


@pytest.mark.parametrize("opt_cls", [RankOneAWeightedPE, DiagonalWeightedPE])
@pytest.mark.parametrize("mode", ["fp32", "comp_bf16", "mixed"])
def test_tiny_gpt_two_steps(device, opt_cls, mode):
    torch.manual_seed(21)
    model = GPT(GPT_TINY)
    model.init_weights(21)
    g = torch.Generator().manual_seed(22)
    batches = []
    for mb in range(3):
        idx = torch.randint(0, GPT_TINY.vocab, (2 + mb, GPT_TINY.ctx), generator=g)
        tgt = torch.randint(0, GPT_TINY.vocab, (2 + mb, GPT_TINY.ctx), generator=g)
        batches.append((idx, tgt))
    loss = lambda m, x, y: m(x, y) / 3
    hist, opt, ora = run_pair(device, model, batches, loss, opt_cls, mode, 3e-3, steps=2,
                              module_filter=transformer_filter)
    # q/k/v share the q activation statistic (sandmuon/optimizer.py:128-135)
    blk = opt.named_matrices
    assert opt.a_sources[id(blk["transformer.h.0.attn.k_proj.weight"])] is blk["transformer.h.0.attn.q_proj.weight"]
    assert "a_ema" not in opt.state[blk["transformer.h.0.attn.k_proj.weight"]]
    worst = check_directions(hist, opt, 3e-3, mode)
    print(f"tiny gpt {opt_cls.__name__} {mode}: worst direction rel err {worst:.3e}")
    check_aux(hist, opt, ora)


def _tiny_gpt_batches(seed, n=3):
    g = torch.Generator().manual_seed(seed)
    out = []
    for mb in range(n):
        idx = torch.randint(0, GPT_TINY.vocab, (2 + mb, GPT_TINY.ctx), generator=g)
        tgt = torch.randint(0, GPT_TINY.vocab, (2 + mb, GPT_TINY.ctx), generator=g)
        out.append((idx, tgt))
    return out


@pytest.mark.parametrize("source", ["gpu", "oracle"])
def test_checkpoint_crossloads_between_the_gpu_build_and_the_oracle(device, source):
    """Checkpoint interop: a state_dict() saved by one side after a step is
    loaded by a fresh instance of the other, and the next step matches the
    uninterrupted side to the parity gates (fp32 mode)."""
    mode, lr = "fp32", 3e-3
    torch.manual_seed(31)
    model = GPT(GPT_TINY)
    model.init_weights(31)
    loss = lambda m, x, y: m(x, y) / 3
    pair = Pair(device, model, RankOneAWeightedPE, mode, lr, transformer_filter)
    pair.step(_tiny_gpt_batches(32), loss)
    if source == "gpu":
        saved = pair.opt.state_dict()
        saved = {"state": {k: {n: (v.detach().cpu().clone() if torch.is_tensor(v) else v) for n, v in e.items()}
                           for k, e in saved["state"].items()},
                 "param_groups": copy.deepcopy(saved["param_groups"])}
        cpu_model = copy.deepcopy(pair.cpu_model)
        ora = O.OracleOptimizer(cpu_model, lr, rank_one_a=True, module_filter=transformer_filter, hooks=False)
        ora.load_state_dict(saved)
        pair.cpu_model, pair.ora = cpu_model, ora
    else:
        saved = pair.ora.state_dict()
        pair.opt.close()
        pair.opt = RankOneAWeightedPE(pair.gpu_model, lr, module_filter=transformer_filter, s8_mode=mode)
        pair.opt.load_state_dict(copy.deepcopy(saved))
        assert all(isinstance(s["step"], int) for s in pair.ora.state.values() if "step" in s)
    entry = pair.step(_tiny_gpt_batches(33), loss)
    check_directions([entry], pair.opt, lr, mode)
    check_aux([entry], pair.opt, pair.ora)
    pair.close()
