"""CPU oracle for the SandMuon optimizer step -- TEST INFRASTRUCTURE ONLY.

This module is a from-scratch eager restatement, on the CPU, of the portable
reference path ``sandmuon/optimizer.py`` (pxike/SandMuon).  It is the checker
that the HIP build is compared against; it is never the thing measured or
shipped.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it.  The product package
(``sandmuon_amd``) never imports it and has no CPU fallback.

Every function names the reference lines it restates.  Arithmetic runs in the
dtype of its inputs: float32 restates the reference's own eager FP32 path,
float64 gives an error yardstick.

Pinning (what checks each function independently of this restatement) is
listed per function under "pinned by"; the tests live in
``tests/test_oracle_pins.py`` and ``tests/test_golden.py``.
"""
from __future__ import annotations

import math
import re
from typing import Callable, Dict, Optional

import torch
from torch import nn

# Fixed S8 recipe: sandmuon/coefficients.py:3-11 (second pin:
# reproduction/paper/s8/data/completed/s8_manifest.json:79-108).
S8_MARGIN = 1.35
S8_MULTIPLIER = 1.0
S8_COEFFICIENTS = (
    (11.062126275847973, -56.051653229128085, 72.32081107619855),
    (4.100720073616268, -2.9324183165353577, 0.5339692084282731),
    (3.930310192522361, -2.873509793709714, 0.5366557527206212),
    (3.280567968245866, -2.414925589994015, 0.48635134757825227),
    (2.282741575232451, -1.6302296637355072, 0.40275720810675486),
)
STATISTIC_BETA = 0.97


def _tiny(dtype: torch.dtype) -> float:
    return torch.finfo(dtype).tiny


# ---------------------------------------------------------------- factors ---
def diagonal_inverse_sqrt(value: torch.Tensor) -> torch.Tensor:
    """Mean-normalised diagonal inverse square root.

    Restates sandmuon/optimizer.py:19-24.  Pinned by: closed form
    (elementwise rsqrt of value/mean with the two clamps), zero-signal
    finiteness (tests/test_optimizer.py:149).
    """
    m = value.mean()
    ratio = torch.maximum(value, m * 1e-6) / torch.clamp(m, min=_tiny(value.dtype))
    return torch.rsqrt(torch.clamp(ratio, min=1e-6))


def rank1_inverse_sqrt(second: torch.Tensor, mean: torch.Tensor):
    """Diagonal D^-1/2 and the Sherman-Morrison rank-one (z, kappa).

    Restates sandmuon/optimizer.py:27-35.  Pinned by: the dense covariance
    identity W (A/q) W^T = I (tests/test_optimizer.py:24-33).
    """
    q = torch.clamp(second.mean(), min=_tiny(second.dtype))
    var = torch.clamp(second - mean * mean, min=0.0)
    inv = torch.rsqrt(torch.clamp(var / q, min=1e-6))
    z = inv * (mean / torch.sqrt(q))
    rho = torch.sqrt(1.0 + (z * z).sum())
    kappa = -1.0 / (rho * (rho + 1.0))
    return inv, z, kappa


# ------------------------------------------------------ whiten / mapback ---
def rank1_whiten(matrix: torch.Tensor, left, right) -> torch.Tensor:
    """V = S*(li x ri); V += lc lz (lz^T V); V += rc (V rz) rz^T.

    Restates sandmuon/optimizer.py:38-45 (batched over leading dims).  Pinned
    by: dense L M R^T oracle (tests/test_optimizer.py:35-43).
    """
    li, lz, lc = left
    ri, rz, rc = right
    v = matrix * li.unsqueeze(-1) * ri.unsqueeze(-2)
    col = torch.matmul(lz.unsqueeze(-2), v)                 # [..., 1, c]
    v = v + lc[..., None, None] * lz.unsqueeze(-1) * col
    row = torch.matmul(v, rz.unsqueeze(-1))                 # [..., r, 1]
    v = v + rc[..., None, None] * row * rz.unsqueeze(-2)
    return v


def rank1_mapback(value: torch.Tensor, left, right) -> torch.Tensor:
    """Rank-one actions (left, then right), then the two diagonals.

    Restates sandmuon/optimizer.py:48-60.  Pinned by: dense
    diag(li)(I+lc lz lz^T) Q (I+rc rz rz^T) diag(ri) (tests/test_optimizer.py:46-54).
    """
    li, lz, lc = left
    ri, rz, rc = right
    v = value + lc * torch.outer(lz, lz @ value)
    v = v + rc * torch.outer(v @ rz, rz)
    return v * li[:, None] * ri[None, :]


def graft_direction(value: torch.Tensor, output_rows: int) -> torch.Tensor:
    """Scale to Frobenius norm sqrt(output_rows).

    Restates sandmuon/optimizer.py:63-66.  Pinned by: the norm invariant
    ||dW||/lr = sqrt(rows) (tests/test_optimizer.py:215-237).
    """
    v = value.float() if value.dtype != torch.float64 else value
    n = torch.clamp(torch.linalg.vector_norm(v), min=_tiny(torch.float32))
    return v * (math.sqrt(float(output_rows)) / n)


# ------------------------------------------------------------------- S8 ---
def s8(x: torch.Tensor, coefficients=S8_COEFFICIENTS, margin=S8_MARGIN,
       multiplier=S8_MULTIPLIER) -> torch.Tensor:
    """Eager S8 polar map in the dtype of ``x`` (float32 restates the reference).

    Restates sandmuon/optimizer.py:69-93: orient rows<=cols, whole-batch zero
    early exit, Frobenius normalisation, stage 1 with the Schatten-8 scale
    s = max(margin*||(XX^T)^2||_F^(1/4), 1e-30), P = a I + b G/s^2 + c G2/s^4,
    X = (P X)/s, then four unscaled stages, transpose back, times multiplier.
    Pinned by: the SVD oracle ``s8_svd`` (closed form U f(S) V^T), the
    orientation/zero invariants (tests/test_optimizer.py:140-149) and
    golden vectors written by the reference itself (tests/golden/).
    """
    flip = x.shape[-2] > x.shape[-1]
    if flip:
        x = x.transpose(-2, -1)
    dtype = x.dtype if x.dtype == torch.float64 else torch.float32
    x = x.to(dtype)
    if not bool(torch.any(x != 0)):
        out = torch.zeros_like(x)
        return out.transpose(-2, -1) if flip else out
    fro = torch.clamp(torch.linalg.matrix_norm(x, keepdim=True), min=1e-30)
    x = x / fro
    eye = torch.eye(x.shape[-2], dtype=dtype)
    g = x @ x.transpose(-2, -1)
    g2 = g @ g
    s = torch.clamp(margin * torch.linalg.matrix_norm(g2, keepdim=True) ** 0.25, min=1e-30)
    a, b, c = coefficients[0]
    p = a * eye + b * g / (s * s) + c * g2 / s ** 4
    x = (p @ x) / s
    for a, b, c in coefficients[1:]:
        g = x @ x.transpose(-2, -1)
        g2 = g @ g
        x = (a * eye + b * g + c * g2) @ x
    if flip:
        x = x.transpose(-2, -1)
    return x * multiplier


def s8_scalar(sigma: torch.Tensor, sensor: torch.Tensor,
              coefficients=S8_COEFFICIENTS, margin=S8_MARGIN) -> torch.Tensor:
    """Scalar composition f(sigma) of the five S8 stages.

    ``sensor`` is the Schatten-8 norm of the (unnormalised) input, i.e.
    (sum sigma^8)^(1/8); the Frobenius prescale cancels in exact arithmetic.
    For X = U diag(sigma) V^T every stage maps singular values through the
    odd polynomial p(t) = t*(a + b t^2 + c t^4).
    """
    t = sigma / (margin * sensor)
    for a, b, c in coefficients:
        t2 = t * t
        t = t * (a + b * t2 + c * t2 * t2)
    return t


def s8_svd(x: torch.Tensor, coefficients=S8_COEFFICIENTS, margin=S8_MARGIN,
           multiplier=S8_MULTIPLIER) -> torch.Tensor:
    """Closed-form S8 through the SVD, in float64: U f(S) V^T.

    Independent of the GEMM order of ``s8``; used to pin it.
    """
    x = x.to(torch.float64)
    u, sv, vh = torch.linalg.svd(x, full_matrices=False)
    sensor = (sv ** 8).sum(-1, keepdim=True) ** 0.125
    f = s8_scalar(sv, sensor, coefficients, margin)
    return (u * f.unsqueeze(-2)) @ vh * multiplier


# --------------------------------------------------------------- stats ---
def accumulate_rows(rows: torch.Tensor, sum_sq: torch.Tensor,
                    sum_first: Optional[torch.Tensor]) -> int:
    """Forward/cotangent hook body: sum_sq += sum_n x^2, sum_first += sum_n x.

    Restates sandmuon/optimizer.py:156-168 (A side) and :171-177 (B side).
    Pinned by: float64 brute-force column sums and the analytic
    microbatch expectations of tests/test_optimizer.py:57-85.
    """
    r = rows.reshape(-1, rows.shape[-1]).to(sum_sq.dtype)
    sum_sq.add_((r * r).sum(0))
    if sum_first is not None:
        sum_first.add_(r.sum(0))
    return r.shape[0]


def finish_a(state: dict, rank_one: bool, beta: float = STATISTIC_BETA):
    """Count-normalise, EMA (first step copies), factor, zero the sums.

    Restates sandmuon/optimizer.py:182-207.
    """
    count = state["a_count"]
    second = state["a_sum"] / count
    if rank_one:
        mean = state["a_first_sum"] / count
        if "a_ema" not in state:
            state["a_ema"] = second.clone()
            state["a_mean_ema"] = mean.clone()
        else:
            state["a_ema"].mul_(beta).add_(second, alpha=1 - beta)
            state["a_mean_ema"].mul_(beta).add_(mean, alpha=1 - beta)
        factor = rank1_inverse_sqrt(state["a_ema"], state["a_mean_ema"])
        state["a_first_sum"].zero_()
    else:
        if "a_ema" not in state:
            state["a_ema"] = second.clone()
        else:
            state["a_ema"].mul_(beta).add_(second, alpha=1 - beta)
        factor = diagonal_inverse_sqrt(state["a_ema"])
    state["a_sum"].zero_()
    state["a_count"] = 0
    return factor, count


def finish_b(state: dict, count: int, beta: float = STATISTIC_BETA):
    """Relative cotangent shape b/mean(b), EMA, diagonal factor, zero sums.

    Restates sandmuon/optimizer.py:209-222.
    """
    b = state["b_sum"] / count
    b = b / torch.clamp(b.mean(), min=_tiny(b.dtype))
    if "b_ema" not in state:
        state["b_ema"] = b.clone()
    else:
        state["b_ema"].mul_(beta).add_(b, alpha=1 - beta)
    inv = diagonal_inverse_sqrt(state["b_ema"])
    state["b_sum"].zero_()
    state["b_count"] = 0
    return inv


def nesterov(momentum: torch.Tensor, grad: torch.Tensor, beta: float) -> torch.Tensor:
    """m <- beta m + (1-beta) g (in place); source = beta m + (1-beta) g.

    Restates sandmuon/optimizer.py:244-248.  Pinned by: closed form.
    """
    momentum.mul_(beta).add_(grad, alpha=1 - beta)
    return momentum * beta + grad * (1 - beta)


def adamw(param, grad, state, lr, betas=(.9, .999), eps=1e-8, weight_decay=.01):
    """Manual AdamW with integer step, decoupled decay before the update.

    Restates sandmuon/optimizer.py:268-281 (lr here is group lr * 0.1).
    Pinned by: torch.optim.AdamW on the CPU (a library routine).
    """
    if "exp_avg" not in state:
        state["exp_avg"] = torch.zeros_like(param, dtype=torch.float32)
        state["exp_avg_sq"] = torch.zeros_like(param, dtype=torch.float32)
        state["step"] = 0
    state["step"] += 1
    b1, b2 = betas
    state["exp_avg"].mul_(b1).add_(grad, alpha=1 - b1)
    state["exp_avg_sq"].mul_(b2).addcmul_(grad, grad, value=1 - b2)
    bc1, bc2 = 1 - b1 ** state["step"], 1 - b2 ** state["step"]
    upd = (state["exp_avg"] / bc1) / ((state["exp_avg_sq"] / bc2).sqrt() + eps)
    param.mul_(1 - lr * weight_decay)
    param.add_(upd.to(param.dtype), alpha=-lr)


# ------------------------------------------------ compensated-BF16 model ---
def _bf16(t: torch.Tensor) -> torch.Tensor:
    """Round to BF16 (nearest even) and back to the working dtype."""
    return t.to(torch.bfloat16).to(t.dtype)


def _split(t: torch.Tensor):
    """hi = bf16(t), lo = bf16(t - hi): the two halves of a stored operand.

    Pinned by: |t - hi - lo| <= 2^-16 |t| and hi, lo BF16-representable
    (tests/test_oracle_pins.py).
    """
    hi = _bf16(t)
    return hi, _bf16(t - hi)


def _stored(t: torch.Tensor) -> torch.Tensor:
    """An operand as the compensated mode stores it between phases: the BF16
    pair hi + lo of each element (16-17 significant bits)."""
    hi, lo = _split(t)
    return hi + lo


def _mm_comp(a: torch.Tensor, b: torch.Tensor, comp: bool = True) -> torch.Tensor:
    """A product as the compensated MFMA path forms it from the hi/lo halves
    of both operands: hi*lo + lo*hi + hi*hi (comp), or hi*hi alone (a plain
    BF16 product).  Products are summed in float64 and rounded once to the
    working dtype, which bounds (does not reproduce) the FP32 accumulation
    order of the MFMAs.

    Follows reproduction/odl/ops/bf16_compensated_mm_fast.py:60-66 (the
    hi/lo split and the three products).  Pinned by: the elementwise bound
    |comp - a b| <= 2^-16 (|a| |b|) against the float64 product, which a
    dropped correction product fails, and the identity case below.
    """
    ah, al = _split(a)
    bh, bl = _split(b)
    acc = ah.double() @ bh.double()
    if comp:
        acc = acc + ah.double() @ bl.double() + al.double() @ bh.double()
    return acc.to(a.dtype)


def _f16(t: torch.Tensor) -> torch.Tensor:
    """Round to FP16 (nearest even, gradual underflow) and back."""
    return t.to(torch.float16).to(t.dtype)


def _mm_f16(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """A product of FP16 operands with a wide accumulator (the FP16 MFMA of
    the mixed mode), rounded once to the working dtype.  Pinned by: the
    elementwise bound |p - a b| <= 2^-10 (|a| |b|) and the identity case."""
    return (_f16(a).double() @ _f16(b).double()).to(a.dtype)


def s8_comp_bf16_model(x: torch.Tensor, comp_stages: int = 5, coefficients=S8_COEFFICIENTS,
                       margin=S8_MARGIN, mask: Optional[int] = None, fp16_stages=()) -> torch.Tensor:
    """Rounding model of the BF16-class S8 of the HIP build (X-space
    schedule): each stage compensated, plain BF16 or FP16.

    Stage k is FP16 if k is in ``fp16_stages`` (the mixed mode: stages
    2-5), else compensated if bit k-1 of ``mask`` is set (default: the first
    ``comp_stages`` stages), else plain BF16.  Follows the build's dataflow:
    every GEMM operand is stored in the form of the stage that reads it (the
    BF16 pair hi + lo, 16-17 significant bits, or FP16); stage 1 scales the
    Gram by 1/||V||^2 and the apply by 1/(||V|| s); G2 of stage 1 and the
    last stage's output stay in the working dtype; stages 2-5 form
    P = c (G G + (b/c) G) + a I with the (b/c) G term as a product of its
    own, whose scalar keeps its hi and lo halves (BF16 or FP16) in every
    form.  A compensated stage uses hi*lo + lo*hi + hi*hi for every product,
    a plain one hi*hi (so comp_stages = 1 is the recipe of
    reproduction/odl/ops/dense_s8_compensated_fast.py:53-85: a BF16 input to
    the plain stages, a compensated stage 1).  The working dtype is the
    input's (float32 models the build; float64 with the roundings replaced
    by the identity reduces it to the exact map, which pins the stage
    algebra against ``s8_svd``).  Used to budget the recipes' error against
    the 1e-2 gate; the GPU measurement is what decides the recipe.
    Pinned by: tests/test_oracle_pins.py (identity case vs the SVD form for
    several recipes, the product bounds and a planted dropped correction
    product).
    """
    wd = x.dtype if x.dtype == torch.float64 else torch.float32
    x = x.to(wd)
    flip = x.shape[-2] > x.shape[-1]
    if flip:
        x = x.transpose(-2, -1)
    if mask is None:
        mask = (1 << comp_stages) - 1
    form = ["f16" if k + 1 in fp16_stages else "comp" if (mask >> k) & 1 else "plain"
            for k in range(len(coefficients))]

    def stored(t, f):
        return _f16(t) if f == "f16" else _stored(t)

    def mm(a, b, f):
        return _mm_f16(a, b) if f == "f16" else _mm_comp(a, b, f == "comp")

    def lin(scalar, g, f):
        """scalar * G as the one-hot MFMAs form it: the scalar's hi and lo
        halves against G (both halves of G when compensated)."""
        if f == "f16":
            sh = _f16(torch.tensor(scalar, dtype=wd))
            sl = _f16(torch.tensor(scalar, dtype=wd) - sh)
            return ((sh.double() + sl.double()) * _f16(g).double()).to(wd)
        sh, sl = _split(torch.tensor(scalar, dtype=wd))
        gh, gl = _split(g)
        acc = sh.double() * gh.double() + sl.double() * gh.double()
        if f == "comp":
            acc = acc + sh.double() * gl.double()
        return acc.to(wd)

    eye = torch.eye(x.shape[-2], dtype=wd)
    fro2 = (x.double() ** 2).sum((-2, -1), keepdim=True)
    xs = _stored(x)
    inv_n2 = torch.where(fro2 > 0, 1.0 / fro2.clamp_min(1e-300), torch.zeros_like(fro2)).to(wd)
    g = _stored(mm(xs, xs.transpose(-2, -1), form[0]) * inv_n2)
    g2 = mm(g, g, form[0])
    s = torch.clamp(margin * torch.linalg.matrix_norm(g2.double(), keepdim=True) ** 0.25, min=1e-30)
    a, b, c = coefficients[0]
    s2 = (s * s).to(wd)
    p = _stored(a * eye + (b * g) / s2 + (c * g2) / (s2 * s2))
    scale = torch.where(fro2 > 0, 1.0 / (fro2.sqrt() * s).clamp_min(1e-300), torch.zeros_like(fro2)).to(wd)
    xk = mm(p, xs, form[0]) * scale
    for k in range(1, len(coefficients)):
        a, b, c = coefficients[k]
        f = form[k]
        xk = stored(xk, f)
        g = stored(mm(xk, xk.transpose(-2, -1), f), f)
        acc = mm(g, g, f) + lin(b / c, g, f)
        p = stored(c * acc + a * eye, f)
        xk = mm(p, xk, f)
    if flip:
        xk = xk.transpose(-2, -1)
    return xk


# --------------------------------------------------------- full optimizer ---
_QKV = re.compile(r"^(transformer\.h\.\d+\.attn\.)[kv]_proj\.weight$")


class OracleOptimizer:
    """CPU restatement of DiagonalWeightedPE / RankOneAWeightedPE.

    Restates sandmuon/optimizer.py:96-328: matrix selection (:106-118),
    q/k/v A-sharing (:128-135), auxiliary AdamW group (:137-144), hooks
    (:151-180), step (:224-316).  Not an optimizer for production use: it
    is the end-to-end checker and the CPU baseline.
    """

    def __init__(self, model: nn.Module, lr: float, *, rank_one_a: bool = True,
                 module_filter: Optional[Callable[[str, nn.Module], bool]] = None,
                 s8_fn: Callable[[torch.Tensor], torch.Tensor] = s8, hooks: bool = True):
        choose = module_filter or (lambda name, module: isinstance(module, nn.Linear))
        self.matrices: Dict[str, nn.Parameter] = {}
        self.modules: Dict[str, nn.Module] = {}
        for name, module in model.named_modules():
            if not name or not choose(name, module):
                continue
            w = getattr(module, "weight", None)
            if isinstance(w, nn.Parameter) and w.requires_grad and w.ndim == 2:
                self.matrices[name + ".weight"] = w
                self.modules[name + ".weight"] = module
        if not self.matrices:
            raise ValueError("No eligible trainable linear weights found")
        self.rank_one = rank_one_a
        self.lr = float(lr)
        self.momentum = .8
        self.s8_fn = s8_fn
        self.names = {id(p): n for n, p in self.matrices.items()}
        self.a_source = {id(p): p for p in self.matrices.values()}
        for name, p in self.matrices.items():
            m = _QKV.match(name)
            if m and (m.group(1) + "q_proj.weight") in self.matrices:
                self.a_source[id(p)] = self.matrices[m.group(1) + "q_proj.weight"]
        ids = {id(p) for p in self.matrices.values()}
        self.aux = [p for p in model.parameters() if p.requires_grad and id(p) not in ids]
        self.state: Dict[int, dict] = {}
        self.handles = [mod.register_forward_hook(self._hook(self.matrices[n]))
                        for n, mod in self.modules.items()] if hooks else []

    def feed(self, name: str, x: Optional[torch.Tensor] = None,
             delta: Optional[torch.Tensor] = None) -> None:
        """Drive the hook bodies with captured tensors instead of a forward."""
        p = self.matrices[name]
        s = self.st(p)
        with torch.no_grad():
            if x is not None and self.a_source[id(p)] is p:
                if "a_sum" not in s:
                    s["a_sum"] = torch.zeros(x.shape[-1], dtype=torch.float32)
                    s["a_count"] = 0
                    if self.rank_one:
                        s["a_first_sum"] = torch.zeros(x.shape[-1], dtype=torch.float32)
                s["a_count"] += accumulate_rows(x, s["a_sum"], s.get("a_first_sum"))
            if delta is not None:
                if "b_sum" not in s:
                    s["b_sum"] = torch.zeros(delta.shape[-1], dtype=torch.float32)
                    s["b_count"] = 0
                s["b_count"] += accumulate_rows(delta, s["b_sum"], None)

    def st(self, p) -> dict:
        return self.state.setdefault(id(p), {})

    def _hook(self, p):
        own = self.a_source[id(p)] is p

        def hook(module, inputs, output):
            if not (module.training and torch.is_grad_enabled()
                    and isinstance(output, torch.Tensor) and output.requires_grad):
                return
            x = inputs[0].detach()
            s = self.st(p)
            if own:
                if "a_sum" not in s:
                    s["a_sum"] = torch.zeros(x.shape[-1], dtype=torch.float32)
                    s["a_count"] = 0
                    if self.rank_one:
                        s["a_first_sum"] = torch.zeros(x.shape[-1], dtype=torch.float32)
                with torch.no_grad():
                    s["a_count"] += accumulate_rows(x, s["a_sum"], s.get("a_first_sum"))

            def thook(grad):
                if "b_sum" not in s:
                    s["b_sum"] = torch.zeros(grad.shape[-1], dtype=torch.float32)
                    s["b_count"] = 0
                with torch.no_grad():
                    s["b_count"] += accumulate_rows(grad.detach(), s["b_sum"], None)
                return grad
            output.register_hook(thook)
        return hook

    @torch.no_grad()
    def step(self):
        items, a_cache = [], {}
        for p in self.matrices.values():
            if p.grad is None:
                continue
            src = self.a_source[id(p)]
            if id(src) not in a_cache:
                ss = self.st(src)
                if ss.get("a_count", 0) < 1:
                    raise RuntimeError(f"Missing activation statistics: {self.names[id(src)]}")
                a_cache[id(src)] = finish_a(ss, self.rank_one)
            a_fac, count = a_cache[id(src)]
            s = self.st(p)
            if s.get("b_count", 0) != count:
                raise RuntimeError("Missing or mismatched cotangent statistics: "
                                   f"{self.names[id(p)]}; expected {count}, got {s.get('b_count', 0)}")
            inv_b = finish_b(s, count)
            if "momentum_buffer" not in s:
                s["momentum_buffer"] = torch.zeros_like(p, dtype=torch.float32)
            g = p.grad.float()
            source = nesterov(s["momentum_buffer"], g, self.momentum)
            rows, cols = p.shape
            flip = rows > cols
            if self.rank_one:
                diag_b = (inv_b, torch.zeros_like(inv_b), torch.zeros(()))
                left, right = (a_fac, diag_b) if flip else (diag_b, a_fac)
            else:
                left, right = (a_fac, inv_b) if flip else (inv_b, a_fac)
            items.append((p, source.transpose(0, 1) if flip else source, left, right, flip))
        for p in self.aux:
            if p.grad is not None:
                adamw(p, p.grad.float(), self.st(p), self.lr * .1)
        groups: Dict[tuple, list] = {}
        for it in items:
            groups.setdefault(tuple(it[1].shape), []).append(it)
        for entries in groups.values():
            src = torch.stack([e[1] for e in entries])
            if self.rank_one:
                L = [torch.stack([e[2][k] for e in entries]) for k in range(3)]
                R = [torch.stack([e[3][k] for e in entries]) for k in range(3)]
                w = rank1_whiten(src, L, R)
            else:
                L = [torch.stack([e[2] for e in entries])]
                R = [torch.stack([e[3] for e in entries])]
                w = src * L[0][:, :, None] * R[0][:, None, :]
            q = self.s8_fn(w)
            dirs = []
            for i, (p, _, _, _, flip) in enumerate(entries):
                if self.rank_one:
                    v = rank1_mapback(q[i], (L[0][i], L[1][i], L[2][i]),
                                      (R[0][i], R[1][i], R[2][i]))
                else:
                    v = q[i] * L[0][i][:, None] * R[0][i][None, :]
                d = graft_direction(v, p.shape[0])
                dirs.append(d.transpose(0, 1) if flip else d)
            for d, (p, *_rest) in zip(dirs, entries):
                p.add_(d.to(p.dtype), alpha=-self.lr)

    # ------------------------------------------------------ checkpoints ---
    def _params(self):
        return list(self.matrices.values()) + list(self.aux)

    def state_dict(self) -> dict:
        """The torch.optim.Optimizer.state_dict() layout of the reference
        (sandmuon/optimizer.py:137-144 groups; state keyed by the index of
        the parameter in group order: matrices, then auxiliaries)."""
        base = dict(lr=self.lr, use_muon=True, momentum=self.momentum, weight_decay=0.,
                    adamw_lr_ratio=.1, adamw_betas=(.9, .999), adamw_eps=1e-8)
        n = len(self.matrices)
        groups = [dict(base, params=list(range(n)))]
        if self.aux:
            groups.append(dict(base, use_muon=False, weight_decay=.01, params=list(range(n, n + len(self.aux)))))
        state = {}
        for i, p in enumerate(self._params()):
            entry = self.state.get(id(p))
            if entry:
                state[i] = {k: (v.clone() if torch.is_tensor(v) else v) for k, v in entry.items()}
        return {"state": state, "param_groups": groups}

    def load_state_dict(self, sd: dict) -> None:
        """Loads a state_dict() of this layout (from this class or from the
        GPU build); tensors move to the CPU, a tensor AdamW step becomes an
        int."""
        params = self._params()
        total = sum(len(g["params"]) for g in sd["param_groups"])
        if total != len(params):
            raise ValueError(f"checkpoint has {total} parameters, this optimizer {len(params)}")
        self.state = {}
        for i, entry in sd["state"].items():
            p = params[int(i)]
            out = {}
            for k, v in entry.items():
                if torch.is_tensor(v):
                    v = v.detach().cpu().clone()
                    if k == "step":
                        v = int(v.item())
                out[k] = v
            self.state[id(p)] = out
        self.lr = float(sd["param_groups"][0]["lr"])

    def close(self):
        for h in self.handles:
            h.remove()
        self.handles.clear()
