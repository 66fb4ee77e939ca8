"""GPU parity at the BASELINE configurations' full sizes.

* cfg2: the whole isolated-S8 batch (36 x 768^2, 9 x 3072x768, 9 x 768x3072)
  with log-uniform row/column scales, against the eager FP32 restatement.
* cfg5 shapes: S8 on 2048^2, 2048x8192 and 8192x2048 matrices.
* cfg3: statistics through the optimizer's hook bodies on bf16 activations
  [16x1024, 768] and [16x1024, 3072] with N(0, 1e-3) cotangents, 8
  microbatches per step, two steps so that the 0.97 EMA path (not only the
  first-step copy) is compared; q/k/v share the q activation statistic.
* cfg4: one optimizer step of the 103M GPT at its real workload (8
  microbatches of 16 x 1024 tokens, forward and backward under bf16
  autocast; 54 matrices, 39.5M AdamW parameters).  The test takes the hook
  statistics itself in FP64 on the GPU and hands them, with the gradients,
  to the CPU oracle, instead of 32 GB of host copies of the hook inputs.
  With 131,072 tokens every gradient has full rank.
* cfg5: one step of the 2048-wide, 24-layer GPT (144 matrices, 105.7M AdamW
  parameters, the 16 GB workspace) with 4 microbatches of 8 x 1024-token
  synthetic hook inputs of the dtypes a bf16-autocast step hands the hooks;
  every direction, momentum buffer and AdamW parameter against the FP32
  oracle's step from the same weights, gradients and FP64 statistics, the
  update norm of every matrix, the statistics against FP64, and one matrix
  of each shape class against the exact map in FP64.
* FP32 mode's error budget: the reference's eager FP32 path, the same path
  with its two Frobenius norms reduced in FP64, and this build's FP32 mode,
  each against the FP64 map.
* The compensated recipe: the worst error of the compensated-BF16 S8 under
  each compensation mask (which stages are compensated, the rest plain
  BF16; smx_s8_comp_mask) and of the mixed mode (compensated stages 1-2,
  FP16 stages 3-5), on the cfg2 batch, the cfg5 shapes and the cfg4 step.

Gates (north star): statistics/EMA rel. error <= 1e-6; per-matrix direction
rel. Frobenius error <= 1e-4 (fp32 mode), <= 1e-2 (comp_bf16 and mixed).
"""
import pytest
import torch

import copy
import math
import time

from oracle import sandmuon_oracle as O
from sandmuon_amd import RankOneAWeightedPE, _native
from sandmuon_amd.optimizer import _s8_fp32
from sandmuon_amd.workloads import GPT, GPT_103M, GPT_2048, GPTConfig, s8_cfg2_batch, stats_cfg3_tensor, transformer_filter

from test_gpu_optimizer import DIR_TOL, STATS_TOL, rel

pytestmark = pytest.mark.gpu


def per_matrix_rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).flatten(-2).norm(dim=-1) / b.flatten(-2).norm(dim=-1)).tolist()


@pytest.mark.parametrize("mode", ["fp32", "comp_bf16", "mixed"])
def test_s8_full_cfg2_batch(device, mode):
    worst = 0.0
    for seed, shape in ((1002, (36, 768, 768)), (1003, (9, 3072, 768)), (1004, (9, 768, 3072))):
        x = s8_cfg2_batch(seed, *shape)
        out = _s8_fp32(x.to(device), mode=mode)
        errs = per_matrix_rel(out, O.s8(x))
        assert len(errs) == shape[0]
        worst = max(worst, max(errs))
        assert max(errs) <= DIR_TOL[mode], (shape, max(errs))
    print(f"cfg2 {mode}: worst per-matrix rel err {worst:.3e}")


@pytest.mark.parametrize("mode", ["fp32", "comp_bf16", "mixed"])
@pytest.mark.parametrize("shape", [(2, 2048, 2048), (1, 2048, 8192), (1, 8192, 2048)])
def test_s8_cfg5_shapes(device, mode, shape):
    """At K = 2048 the eager FP32 path itself is 1.1e-4 to 1.6e-4 (relative
    Frobenius) away from the FP64 result on these inputs, so a 1e-4 gate
    against it would measure its own rounding.  FP32-MFMA mode is gated at
    1e-4 against the FP64 oracle instead (a stricter bar, which the FP32 path
    itself misses); compensated-BF16 mode keeps its 1e-2 gate against the
    FP32 path."""
    x = s8_cfg2_batch(1005 + shape[1] // 1024 + shape[2], *shape)
    out = _s8_fp32(x.to(device), mode=mode)
    ref32 = O.s8(x)
    errs = per_matrix_rel(out, ref32)
    if mode == "fp32":
        ref64 = O.s8(x.double())
        e_gpu, e_ref = per_matrix_rel(out, ref64), per_matrix_rel(ref32, ref64)
        print(mode, shape, "vs fp64 oracle", e_gpu, "(fp32 oracle vs fp64:", e_ref, "; gpu vs fp32 oracle:", errs, ")")
        assert max(e_gpu) <= DIR_TOL[mode]
    else:
        print(mode, shape, "rel err vs fp32 oracle", errs)
        assert max(errs) <= DIR_TOL[mode]


def _oracle_s8_with_fp64_norms(x):
    """The oracle's eager FP32 S8 (the reference's op order) with its two
    Frobenius norms, ||X|| and ||G2|| (which sets the Schatten scale s),
    reduced in FP64 and rounded to FP32; every GEMM stays FP32."""
    orig = torch.linalg.matrix_norm

    def norm64(t, *args, **kwargs):
        return orig(t.double(), *args, **kwargs).to(t.dtype)
    torch.linalg.matrix_norm = norm64
    try:
        return O.s8(x)
    finally:
        torch.linalg.matrix_norm = orig


@pytest.mark.parametrize("shape", [(1, 768, 768), (1, 768, 3072), (1, 2048, 2048)])
def test_fp32_mode_error_sources(device, shape):
    """Where the FP32-mode error stands against the exact (FP64) map, on cfg2
    inputs.  The reference's eager FP32 path loses most of its accuracy in
    torch's FP32 reduction of ||G2||_F on the CPU: the error of that norm
    moves s, and with only the two norms taken in FP64 the same path lands
    several times closer to FP64.  This build takes s from FP64 tile
    partials, so its FP32-mode error is that of its FP32 GEMMs (an MFMA
    accumulation chain over K).  On the square shapes it is below the
    reference path's own error by 3x (768^2) and 10x (2048^2); on 768 x 3072
    the two are within 1.5x of each other."""
    x = s8_cfg2_batch(2000 + shape[1] + shape[2], *shape)
    ref64 = O.s8(x.double())
    e_ref32 = per_matrix_rel(O.s8(x), ref64)[0]
    e_norm64 = per_matrix_rel(_oracle_s8_with_fp64_norms(x), ref64)[0]
    e_gpu = per_matrix_rel(_s8_fp32(x.to(device), mode="fp32"), ref64)[0]
    print(f"{shape}: vs FP64 map: reference FP32 path {e_ref32:.2e}, with FP64 norms {e_norm64:.2e}, "
          f"this build's FP32 mode {e_gpu:.2e}")
    assert e_norm64 * 3 < e_ref32
    if shape[1] == shape[2]:
        assert e_gpu < e_ref32
    assert e_gpu <= 3e-5


def _cfg3_pool(seed, width, n, cotangent):
    out = []
    for k in range(n):
        if cotangent:
            g = torch.Generator().manual_seed(seed + k)
            t = (torch.randn(16 * 1024, width, generator=g) * 1e-3).bfloat16()
        else:
            t = stats_cfg3_tensor(seed + k, 16 * 1024, width)
        out.append(t)
    return out


def test_cfg3_statistics_through_the_hooks(device):
    cfg = GPTConfig(vocab=97, ctx=16, layers=1, width=768, heads=12, mlp=3072)
    model = GPT(cfg)
    model.init_weights(1003)
    cpu_model = GPT(cfg)
    cpu_model.load_state_dict(model.state_dict())
    model = model.to(device)
    opt = RankOneAWeightedPE(model, 1e-2, module_filter=transformer_filter)
    ora = O.OracleOptimizer(cpu_model, 1e-2, rank_one_a=True, module_filter=transformer_filter, hooks=False)
    names = list(opt.named_matrices)
    assert len(names) == 6
    gp = dict(model.named_parameters())
    pools = {("a", 768): _cfg3_pool(3100, 768, 4, False), ("a", 3072): _cfg3_pool(3200, 3072, 4, False),
             ("b", 768): _cfg3_pool(3300, 768, 4, True), ("b", 3072): _cfg3_pool(3400, 3072, 4, True)}
    on_gpu = {k: [t.to(device) for t in v] for k, v in pools.items()}
    # hook inputs per matrix: (A width or None when the A statistic is shared, B width)
    plan = {"attn.q_proj": (768, 768), "attn.k_proj": (None, 768), "attn.v_proj": (None, 768),
            "attn.c_proj": (768, 768), "mlp.c_fc": (768, 3072), "mlp.c_proj": (3072, 768)}
    g = torch.Generator().manual_seed(1003)
    for step in range(2):
        for mb in range(8):
            for j, (short, (aw, bw)) in enumerate(plan.items()):
                name = f"transformer.h.0.{short}.weight"
                k = (mb + j + step) % 4
                if aw is not None:
                    opt._accumulate_a(gp[name], on_gpu[("a", aw)][k])
                    ora.feed(name, x=pools[("a", aw)][k])
                opt._accumulate_b(gp[name], on_gpu[("b", bw)][(k + 1) % 4])
                ora.feed(name, delta=pools[("b", bw)][(k + 1) % 4])
        for n, p in model.named_parameters():
            grad = torch.randn(p.shape, generator=g) * 1e-3
            p.grad = grad.to(device)
            dict(cpu_model.named_parameters())[n].grad = grad.clone()
        opt.step()
        ora.step()
        torch.cuda.synchronize()
        worst = 0.0
        for n, p in opt.named_matrices.items():
            gs, cs = opt.state[p], ora.st(ora.matrices[n])
            for key in ("a_ema", "a_mean_ema", "b_ema"):
                if key in cs:
                    e = rel(gs[key], cs[key])
                    worst = max(worst, e)
                    assert e <= STATS_TOL, (step, n, key, e)
                else:
                    assert key not in gs, (n, key)
        print(f"cfg3 step {step}: worst statistic rel err {worst:.3e}")
    opt.close()


class Stats64:
    """The hook statistics of every selected matrix, taken by the test itself
    in FP64 on the GPU (sum x^2, sum x and rows of each input; sum delta^2
    and rows of each cotangent), for the same forward/backward passes the
    optimizer's hooks see."""

    def __init__(self, opt):
        self.sums = {}
        self.handles = []
        for name, module in opt._matrix_modules.items():
            self.handles.append(module.register_forward_hook(self._hook(name)))

    def _add(self, key, t, first):
        rows = t.detach().reshape(-1, t.shape[-1]).double()
        e = self.sums.setdefault(key, [0.0, 0.0, 0])
        e[0] = e[0] + rows.square().sum(0)
        if first:
            e[1] = e[1] + rows.sum(0)
        e[2] += rows.shape[0]

    def _hook(self, name):
        def hook(module, inputs, output):
            if not (module.training and torch.is_grad_enabled() and output.requires_grad):
                return
            self._add((name, "a"), inputs[0], True)
            output.register_hook(lambda g: self._add((name, "b"), g, False))
        return hook

    def close(self):
        for h in self.handles:
            h.remove()


def feed_oracle(ora, stats):
    """Oracle state as its hooks would leave it, from FP64 sums (rounded to
    the FP32 of its accumulators)."""
    for name, p in ora.matrices.items():
        st = ora.st(p)
        if ora.a_source[id(p)] is p:
            sq, first, n = stats[(name, "a")]
            st.update(a_sum=sq.float().cpu(), a_first_sum=first.float().cpu(), a_count=n)
        sq, _, n = stats[(name, "b")]
        st.update(b_sum=sq.float().cpu(), b_count=n)


def check_statistics(opt, stats):
    """a_ema, a_mean_ema and b_ema after a first step against FP64."""
    worst = 0.0
    for name, p in opt.named_matrices.items():
        st = opt.state[p]
        if (name, "a") in stats and opt.a_sources[id(p)] is p:
            sq, first, n = stats[(name, "a")]
            for key, want in (("a_ema", sq / n), ("a_mean_ema", first / n)):
                e = rel(st[key], want)
                worst = max(worst, e)
                assert e <= STATS_TOL, (name, key, e)
        sq, _, n = stats[(name, "b")]
        b = sq / n
        e = rel(st["b_ema"], b / b.mean())
        worst = max(worst, e)
        assert e <= STATS_TOL, (name, "b_ema", e)
    return worst


def fp64_direction(st, src, shape, grad, beta=0.8):
    """The update direction of one matrix in FP64 with the oracle's
    functions, from a side's post-step state (`st` of the matrix, `src` of
    its activation-statistic source: the first step's EMAs are the step's
    own statistics, the momentum its updated buffer) and the gradient."""
    d64 = lambda t: t.detach().double().cpu()
    a_fac = O.rank1_inverse_sqrt(d64(src["a_ema"]), d64(src["a_mean_ema"]))
    inv_b = O.diagonal_inverse_sqrt(d64(st["b_ema"]))
    source = d64(st["momentum_buffer"]) * beta + d64(grad) * (1 - beta)
    rows, cols = shape
    flip = rows > cols
    diag_b = (inv_b, torch.zeros_like(inv_b), torch.zeros((), dtype=torch.float64))
    left, right = (a_fac, diag_b) if flip else (diag_b, a_fac)
    s = source.t() if flip else source
    w = O.rank1_whiten(s[None], [t[None] if t.ndim else t.reshape(1) for t in left],
                       [t[None] if t.ndim else t.reshape(1) for t in right])
    q = O.s8(w)[0]
    d = O.graft_direction(O.rank1_mapback(q, left, right), rows)
    return d.t() if flip else d


def directions(before, model, names, lr):
    params = dict(model.named_parameters())
    return {n: ((before[n] - params[n].detach()).double() / lr) for n in names}


def cfg4_run(device, mode):
    """The cfg4 step: GPU model, optimizer and FP64 statistics, the CPU
    oracle holding the same weights, gradients and statistics."""
    model = GPT(GPT_103M)
    model.init_weights(1337)
    cpu_model = copy.deepcopy(model)
    model = model.to(device)
    opt = RankOneAWeightedPE(model, 1e-2, module_filter=transformer_filter, s8_mode=mode)
    stats = Stats64(opt)
    g = torch.Generator(device=device).manual_seed(1337)
    opt.zero_grad(set_to_none=True)
    for _ in range(8):
        idx = torch.randint(0, GPT_103M.vocab, (16, 1024), generator=g, device=device)
        tgt = torch.randint(0, GPT_103M.vocab, (16, 1024), generator=g, device=device)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            loss = model(idx, tgt) / 8
        loss.backward()
    stats.close()
    ora = O.OracleOptimizer(cpu_model, 1e-2, rank_one_a=True, module_filter=transformer_filter, hooks=False)
    feed_oracle(ora, stats.sums)
    with torch.no_grad():
        for (n, p), (_, c) in zip(model.named_parameters(), cpu_model.named_parameters()):
            c.grad = p.grad.detach().cpu().clone()
    return model, cpu_model, opt, ora, stats.sums


# The compensation recipes compared: stages whose bit is set in the mask
# are compensated, the others plain BF16 products (smx_s8_comp_mask).
RECIPES = {"all five": 0x1F, "plain 5": 0x0F, "plain 4": 0x17, "plain 3": 0x1B, "plain 2": 0x1D,
           "plain 2,4": 0x15, "plain 3,4": 0x13, "stage 1 only (historical)": 0x01}


@pytest.mark.parametrize("mode", ["fp32", "comp_bf16", "mixed"])
def test_cfg4_gpt_step_at_the_real_workload(device, mode):
    t0 = time.time()
    model, cpu_model, opt, ora, stats = cfg4_run(device, mode)
    assert len(opt.named_matrices) == 54
    names = list(opt.named_matrices)
    before = {n: p.detach().clone() for n, p in model.named_parameters()}
    grads = {n: p.grad.detach().clone() for n, p in model.named_parameters()}
    sd = copy.deepcopy(opt.state_dict())
    opt.step()
    torch.cuda.synchronize()
    worst_stats = check_statistics(opt, stats)
    t1 = time.time()
    cpu_before = {n: p.detach().clone() for n, p in cpu_model.named_parameters()}
    ora.step()
    t2 = time.time()
    got = directions(before, model, names, 1e-2)
    want = {n: (cpu_before[n] - p.detach()).double() / 1e-2 for n, p in cpu_model.named_parameters() if n in got}
    errs = {n: rel(got[n], want[n]) for n in names}
    worst = max(errs.values())
    for n in names:
        assert torch.isfinite(got[n]).all()
        assert abs(got[n].norm().item() - math.sqrt(before[n].shape[0])) <= 1e-4 * math.sqrt(before[n].shape[0])
    # AdamW on the 39.5M auxiliary parameters, elementwise FP32
    cparams = dict(cpu_model.named_parameters())
    for n, p in model.named_parameters():
        if n not in got:
            assert rel(p, cparams[n]) <= 1e-6, n
    print(f"cfg4 real workload {mode}: worst direction rel err {worst:.3e} (gate {DIR_TOL[mode]}), "
          f"worst statistic {worst_stats:.2e}; GPU part {t1 - t0:.1f}s, oracle step {t2 - t1:.1f}s")
    assert worst <= DIR_TOL[mode], max(errs, key=errs.get)
    if mode == "fp32":
        # The GPU's FP32-MFMA direction and the eager FP32 oracle's, each
        # against the FP64 direction, on one matrix of each shape class.
        for n in ("transformer.h.0.attn.q_proj.weight", "transformer.h.0.mlp.c_fc.weight",
                  "transformer.h.0.mlp.c_proj.weight", "transformer.h.8.attn.v_proj.weight"):
            p, pc = opt.named_matrices[n], ora.matrices[n]
            g64 = fp64_direction(opt.state[p], opt.state[opt.a_sources[id(p)]], p.shape, grads[n])
            o64 = fp64_direction(ora.st(pc), ora.st(ora.a_source[id(pc)]), pc.shape, pc.grad)
            print(f"  {n}: gpu vs fp64 {rel(got[n], g64):.2e}, fp32 oracle vs fp64 {rel(want[n], o64):.2e}, "
                  f"fp64 from either side's statistics {rel(g64, o64):.2e}")
    elif mode == "comp_bf16":
        # The recipe table: the same step from the same state with each
        # compensation mask (plain stages: BF16 products hi*hi).
        table = {}
        try:
            for label, mask in RECIPES.items():
                with torch.no_grad():
                    for n, p in model.named_parameters():
                        p.copy_(before[n])
                opt.load_state_dict(copy.deepcopy(sd))
                _native.s8_comp_mask(mask)
                opt.step()
                torch.cuda.synchronize()
                dk = directions(before, model, names, 1e-2)
                table[label] = max(rel(dk[n], want[n]) for n in names)
        finally:
            _native.s8_comp_mask(0x1F)
        print("cfg4 step, compensation recipe -> worst direction rel err vs the FP32 oracle: " +
              ", ".join(f"{k}: {e:.2e}" for k, e in table.items()))
        assert abs(table["all five"] - worst) <= 1e-6  # the reloaded state repeats the step
    else:
        assert worst <= 5e-3, worst  # the mixed recipe keeps half the gate in reserve
    opt.close()


def test_compensated_stage_recipe_on_cfg2_and_cfg5_shapes(device):
    """Worst per-matrix error against the FP32 oracle of each compensation
    recipe of the compensated-BF16 S8 (plain stages: BF16 products hi*hi)
    and of the mixed mode (compensated stages 1-2, FP16 stages 3-5): the whole
    cfg2 batch and the cfg5 shapes.  The production recipe (all five
    stages) and the mixed mode must stay within half the 1e-2 gate; the
    table is printed for the recipe decision."""
    cases = [((1002, (36, 768, 768)), "cfg2 768x768"), ((1003, (9, 3072, 768)), "cfg2 3072x768"),
             ((1004, (9, 768, 3072)), "cfg2 768x3072"), ((1009, (2, 2048, 2048)), "cfg5 2048x2048"),
             ((1015, (1, 2048, 8192)), "cfg5 2048x8192")]
    table = {}
    try:
        for (seed, shape), label in cases:
            x = s8_cfg2_batch(seed, *shape)
            ref = O.s8(x)
            xd = x.to(device)
            for recipe, mask in RECIPES.items():
                _native.s8_comp_mask(mask)
                table[(label, recipe)] = max(per_matrix_rel(_s8_fp32(xd, mode="comp_bf16"), ref))
            _native.s8_comp_mask(0x1F)
            table[(label, "mixed")] = max(per_matrix_rel(_s8_fp32(xd, mode="mixed"), ref))
    finally:
        _native.s8_comp_mask(0x1F)
    recipes = list(RECIPES) + ["mixed"]
    for _, label in cases:
        print(f"{label}: " + ", ".join(f"{r}: {table[(label, r)]:.2e}" for r in recipes))
    for (label, recipe), e in table.items():
        if recipe in ("all five", "mixed"):
            assert e <= 5e-3, (label, recipe, e)


def _init_on_device(model, seed, device):
    """GPT.init_weights' distributions, drawn on the GPU (1.3B parameters)."""
    g = torch.Generator(device=device).manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if p.ndim == 2:
                std = 0.02 / math.sqrt(2 * model.cfg.layers) if name.endswith("c_proj.weight") else 0.02
                p.normal_(0.0, std, generator=g)
            elif name.endswith(".bias"):
                p.zero_()
            else:
                p.fill_(1.0)


@pytest.mark.parametrize("mode", ["comp_bf16", "mixed"])
def test_cfg5_gpt_step(device, mode):
    """BASELINE cfg5: the 2048-wide GPT's step in compensated-BF16 (and the
    mixed) mode with 4 microbatches of 8 x 1024-token hook inputs
    (LayerNorm-fed q/c_fc inputs in fp32, the attention and GELU outputs and
    every cotangent in bf16, as a bf16-autocast step hands them; two
    rotating input sets)."""
    t0 = time.time()
    cfg = GPT_2048
    with torch.device(device):
        model = GPT(cfg)
    _init_on_device(model, 2048, device)
    lr = 1e-2
    opt = RankOneAWeightedPE(model, lr, module_filter=transformer_filter, s8_mode=mode)
    assert len(opt.named_matrices) == 144
    aux = [p for p in model.parameters() if id(p) not in {id(q) for q in opt.named_matrices.values()}]
    assert sum(p.numel() for p in aux) == 105_666_560
    g = torch.Generator(device=device).manual_seed(5)
    rows, w, m = 8 * 1024, cfg.width, cfg.mlp
    sets = []
    for _ in range(2):
        a, b = [], []
        for blk in model.transformer.h:
            a += [(blk.attn.q_proj.weight, torch.randn(rows, w, generator=g, device=device)),
                  (blk.attn.c_proj.weight, torch.randn(rows, w, generator=g, device=device).bfloat16()),
                  (blk.mlp.c_fc.weight, torch.randn(rows, w, generator=g, device=device) + 0.5),
                  (blk.mlp.c_proj.weight, torch.randn(rows, m, generator=g, device=device).abs().bfloat16())]
            for lin, width in ((blk.attn.q_proj, w), (blk.attn.k_proj, w), (blk.attn.v_proj, w),
                               (blk.attn.c_proj, w), (blk.mlp.c_fc, m), (blk.mlp.c_proj, w)):
                b.append((lin.weight, (torch.randn(rows, width, generator=g, device=device) * 1e-3).bfloat16()))
        sets.append((a, b))
    for p in model.parameters():
        p.grad = torch.randn(p.shape, generator=g, device=device) * 1e-3
    for k in range(4):
        a, b = sets[k % 2]
        for p, x in a:
            opt._accumulate_a(p, x)
        for p, d in b:
            opt._accumulate_b(p, d)
    names = {id(p): n for n, p in model.named_parameters()}
    before = {id(p): p.detach().clone() for p in model.parameters()}
    grads = {n: p.grad.detach().clone() for n, p in opt.named_matrices.items()}
    opt.step()
    torch.cuda.synchronize()
    t1 = time.time()
    # update norm and finiteness of every matrix
    for n, p in opt.named_matrices.items():
        dw = (before[id(p)] - p.detach()).double() / lr
        assert torch.isfinite(dw).all(), n
        assert abs(dw.norm().item() - math.sqrt(p.shape[0])) <= 1e-4 * math.sqrt(p.shape[0]), n
    # statistics against FP64 sums of the same inputs (each set used twice),
    # kept as the oracle's hook state
    worst_stats = 0.0
    stats = {}
    for (pa, x), j in zip(sets[0][0], range(len(sets[0][0]))):
        x1 = sets[1][0][j][1]
        sq = sum(t.double().square().sum(0) for t in (x, x1)) * 2
        first = sum(t.double().sum(0) for t in (x, x1)) * 2
        stats[(names[id(pa)], "a")] = (sq, first, 4 * rows)
        st = opt.state[pa]
        for key, want in (("a_ema", sq / (4 * rows)), ("a_mean_ema", first / (4 * rows))):
            e = rel(st[key], want)
            worst_stats = max(worst_stats, e)
            assert e <= STATS_TOL, (key, e)
    for j, (pb, d) in enumerate(sets[0][1]):
        d1 = sets[1][1][j][1]
        bsq = sum(t.double().square().sum(0) for t in (d, d1)) * 2
        stats[(names[id(pb)], "b")] = (bsq, None, 4 * rows)
        bsum = bsq / (4 * rows)
        e = rel(opt.state[pb]["b_ema"], bsum / bsum.mean())
        worst_stats = max(worst_stats, e)
        assert e <= STATS_TOL, ("b_ema", e)
    del sets
    # The FP32 oracle's step on the CPU from the same weights, gradients and
    # FP64 statistics: all 144 directions, the momentum and every AdamW
    # parameter.
    with torch.device("meta"):
        cpu_model = GPT(cfg)
    cpu_model = cpu_model.to_empty(device="cpu")
    gparams = dict(model.named_parameters())
    with torch.no_grad():
        for n, c in cpu_model.named_parameters():
            gp = gparams[n]
            c.copy_(before[id(gp)].cpu())
            c.grad = gp.grad.detach().cpu()
    ora = O.OracleOptimizer(cpu_model, lr, rank_one_a=True, module_filter=transformer_filter, hooks=False)
    assert list(ora.matrices) == list(opt.named_matrices)
    feed_oracle(ora, stats)
    t2 = time.time()
    print(f"cfg5: GPU step and statistics checked ({t2 - t0:.1f}s); oracle step on the CPU", flush=True)
    ora.step()
    t3 = time.time()
    cparams = dict(cpu_model.named_parameters())
    errs = {}
    for n, p in opt.named_matrices.items():
        got = (before[id(p)] - p.detach()).double().cpu() / lr
        want = (before[id(p)].cpu() - cparams[n].detach()).double() / lr
        errs[n] = rel(got, want)
        assert rel(opt.state[p]["momentum_buffer"], ora.st(ora.matrices[n])["momentum_buffer"]) <= 1e-6, n
    worst = max(errs.values())
    assert worst <= DIR_TOL[mode], (max(errs, key=errs.get), worst)
    worst_aux = 0.0
    for n, p in model.named_parameters():
        if n not in errs:
            e = rel(p, cparams[n])
            worst_aux = max(worst_aux, e)
            assert e <= 1e-6, n
    # one matrix of each shape class against the exact map (FP64, from the
    # oracle's statistics and momentum)
    exact = {}
    blk = "transformer.h.0."
    for n in (blk + "attn.q_proj.weight", blk + "mlp.c_fc.weight", blk + "mlp.c_proj.weight"):
        p, pc = opt.named_matrices[n], ora.matrices[n]
        got = (before[id(p)] - p.detach()).double().cpu() / lr
        exact[n] = rel(got, fp64_direction(ora.st(pc), ora.st(ora.a_source[id(pc)]), pc.shape, grads[n]))
        assert exact[n] <= DIR_TOL[mode], (n, exact[n])
    print(f"cfg5 step ({mode}): 144 matrices, worst direction rel err vs the FP32 oracle {worst:.3e} "
          f"({max(errs, key=errs.get)}), statistics worst {worst_stats:.2e}, AdamW worst {worst_aux:.2e}; "
          "FP64 directions " + ", ".join(f"{n.split('.', 3)[-1]} {e:.2e}" for n, e in exact.items())
          + f"; GPU part {t1 - t0:.1f}s, oracle step {t3 - t2:.1f}s, total {time.time() - t0:.1f}s")
    opt.close()
