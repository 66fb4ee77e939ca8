"""Write golden vectors by running the reference's portable path (pxike/SandMuon,
sandmuon/optimizer.py) on the CPU of the build container.

    PYTHONDONTWRITEBYTECODE=1 python tests/golden/make_golden.py /root/reference

The closed forms and invariants in tests/test_oracle_pins.py pin every
oracle function except three things only the reference itself can fix:
  1. _s8_fp32's own FP32 rounding order (s8_fp32.npz),
  2. the end-to-end composition of step(): statistics -> EMA -> factors ->
     momentum -> whiten -> S8 -> mapback -> graft -> W, plus AdamW
     (step_rank1.npz, step_diag.npz),
  3. the structure of state_dict() (state_dict.json).
Inputs come from numpy PCG64 (stable across torch versions) and are stored
next to the outputs.  Fixtures are plain .npz/.json (no pickles).  The
reference is only imported here, in the build container; nothing under
tests/ reads /root/reference at test time.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from sandmuon_amd.workloads import GPT, GPT_TINY, transformer_filter  # noqa: E402


def pcg(seed):
    return np.random.Generator(np.random.PCG64(seed))


def cfg2_like(seed, shape):
    r = pcg(seed)
    b, m, n = shape
    x = r.standard_normal(shape)
    x *= np.exp(r.uniform(np.log(1e-2), np.log(1e2), (b, m, 1)))
    x *= np.exp(r.uniform(np.log(1e-2), np.log(1e2), (b, 1, n)))
    return x.astype(np.float32)


def tiny_model(seed):
    r = pcg(seed)
    model = GPT(GPT_TINY)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if p.ndim == 2:
                p.copy_(torch.from_numpy(r.normal(0, 0.02, p.shape).astype(np.float32)))
            elif name.endswith(".bias"):
                p.copy_(torch.from_numpy(r.normal(0, 0.01, p.shape).astype(np.float32)))
            else:
                p.copy_(torch.from_numpy(1 + r.normal(0, 0.05, p.shape).astype(np.float32)))
    return model


def tokens(seed, n_micro):
    r = pcg(seed)
    out = []
    for mb in range(n_micro):
        b = 2 + mb  # uneven microbatches
        out.append((r.integers(0, GPT_TINY.vocab, (b, GPT_TINY.ctx)), r.integers(0, GPT_TINY.vocab, (b, GPT_TINY.ctx))))
    return out


def run_steps(opt_cls, model, batches, steps, lr):
    opt = opt_cls(model, lr=lr, module_filter=transformer_filter)
    snaps = []
    for _ in range(steps):
        opt.zero_grad(set_to_none=True)
        for idx, tgt in batches:
            (model(torch.from_numpy(idx), torch.from_numpy(tgt)) / len(batches)).backward()
        opt.step()
        snaps.append({n: p.detach().numpy().copy() for n, p in model.named_parameters()})
    return opt, snaps


def main(reference: str) -> None:
    sys.path.insert(0, reference)
    from sandmuon.optimizer import DiagonalWeightedPE, RankOneAWeightedPE, _s8_fp32

    torch.manual_seed(0)
    # 1. S8 FP32 rounding of the reference op order.
    s8 = {}
    for k, shape in enumerate([(2, 64, 96), (2, 96, 64), (1, 128, 128)]):
        x = cfg2_like(2000 + k, shape)
        s8[f"x{k}"] = x
        s8[f"y{k}"] = _s8_fp32(torch.from_numpy(x)).numpy()
    np.savez_compressed(HERE / "s8_fp32.npz", **s8)

    # 2. End-to-end step composition on a tiny GPT (two steps, rank-one;
    #    one step, diagonal).
    for tag, cls, steps in (("rank1", RankOneAWeightedPE, 2), ("diag", DiagonalWeightedPE, 1)):
        model = tiny_model(3000)
        init = {n: p.detach().numpy().copy() for n, p in model.named_parameters()}
        batches = tokens(3001, 3)
        opt, snaps = run_steps(cls, model, batches, steps, lr=3e-3)
        out = {f"init/{n}": v for n, v in init.items()}
        for i, (idx, tgt) in enumerate(batches):
            out[f"idx/{i}"], out[f"tgt/{i}"] = idx, tgt
        for s, snap in enumerate(snaps):
            out.update({f"step{s + 1}/{n}": v for n, v in snap.items()})
        names = {id(p): n for n, p in model.named_parameters()}
        for p, st in opt.state.items():
            for key, val in st.items():
                if isinstance(val, torch.Tensor):
                    out[f"state/{names[id(p)]}/{key}"] = val.numpy().copy()
                else:
                    out[f"state/{names[id(p)]}/{key}"] = np.asarray(val)
        np.savez_compressed(HERE / f"step_{tag}.npz", **out)
        if tag == "rank1":
            sd = opt.state_dict()
            struct = {
                "param_groups": [{k: (v if k != "params" else len(v)) for k, v in g.items()} for g in sd["param_groups"]],
                "state": {str(i): {k: ({"tensor": list(v.shape), "dtype": str(v.dtype)} if isinstance(v, torch.Tensor)
                                       else {"type": type(v).__name__})
                                   for k, v in st.items()} for i, st in sd["state"].items()},
            }
            (HERE / "state_dict.json").write_text(json.dumps(struct, indent=1, sort_keys=True))
        opt.close()
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")), "state_dict.json")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
