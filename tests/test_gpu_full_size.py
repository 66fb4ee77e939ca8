"""GPU parity at the BASELINE configurations' full sizes.

* cfg2: the whole isolated-S8 batch (36 x 768^2, 9 x 3072x768, 9 x 768x3072)
  with log-uniform row/column scales, against the eager FP32 restatement.
* cfg5 shapes: S8 on 2048^2, 2048x8192 and 8192x2048 matrices.
* cfg3: statistics through the optimizer's hook bodies on bf16 activations
  [16x1024, 768] and [16x1024, 3072] with N(0, 1e-3) cotangents, 8
  microbatches per step, two steps so that the 0.97 EMA path (not only the
  first-step copy) is compared; q/k/v share the q activation statistic.
* cfg4: one optimizer step of the 103M GPT (54 matrices at their real
  shapes, 39.5M AdamW parameters), with the hook inputs of two 1024-token
  microbatches, against the CPU oracle fed the same tensors.

Gates (north star): statistics/EMA rel. error <= 1e-6; per-matrix direction
rel. Frobenius error <= 1e-4 (fp32 mode), <= 1e-2 (comp_bf16 mode).
"""
import pytest
import torch

from oracle import sandmuon_oracle as O
from sandmuon_amd import RankOneAWeightedPE
from sandmuon_amd.optimizer import _s8_fp32
from sandmuon_amd.workloads import GPT, GPT_103M, GPTConfig, s8_cfg2_batch, stats_cfg3_tensor, transformer_filter

from test_gpu_optimizer import DIR_TOL, STATS_TOL, check_aux, check_directions, rel, run_pair

pytestmark = pytest.mark.gpu


def per_matrix_rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).flatten(-2).norm(dim=-1) / b.flatten(-2).norm(dim=-1)).tolist()


@pytest.mark.parametrize("mode", ["fp32", "comp_bf16"])
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


@pytest.mark.parametrize("mode", ["fp32", "comp_bf16"])
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


@pytest.mark.parametrize("mode", ["fp32", "comp_bf16"])
def test_cfg4_gpt_step_at_full_shapes(device, mode):
    """Two microbatches of 1024 tokens: with fewer rows than the matrices'
    768 columns every gradient is rank-deficient (condition numbers of
    1e10-1e12 at 2 x 128 tokens), and on such inputs the FP32 S8 of the
    reference is itself ~1e-4 away from the exact map, the size of the gate."""
    model = GPT(GPT_103M)
    model.init_weights(1337)
    g = torch.Generator().manual_seed(1337)
    batches = [(torch.randint(0, GPT_103M.vocab, (1, 1024), generator=g),
                torch.randint(0, GPT_103M.vocab, (1, 1024), generator=g)) for _ in range(2)]
    loss = lambda m, x, y: m(x, y) / 2
    hist, opt, ora = run_pair(device, model, batches, loss, RankOneAWeightedPE, mode, 1e-2, steps=1,
                              module_filter=transformer_filter)
    assert len(opt.named_matrices) == 54
    worst = check_directions(hist, opt, 1e-2, mode)
    print(f"cfg4 {mode}: worst direction rel err {worst:.3e}")
    check_aux(hist, opt, ora)
