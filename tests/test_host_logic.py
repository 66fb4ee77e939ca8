"""Host-side logic of the drop-in API that runs without a GPU: matrix
selection, q/k/v sharing, constructor errors and the loud failure on CPU
parameters (the HIP library is the only compute path)."""
import pytest
import torch
from torch import nn

from sandmuon_amd import DiagonalWeightedPE, RankOneAWeightedPE, S8_COEFFICIENTS, S8_MARGIN, S8_MULTIPLIER
from sandmuon_amd.optimizer import select_matrices, shared_source
from sandmuon_amd.workloads import GPT, GPT_103M, transformer_filter


class Attention(nn.Module):
    def __init__(self):
        super().__init__()
        self.q_proj = nn.Linear(4, 4, bias=False)
        self.k_proj = nn.Linear(4, 4, bias=False)
        self.v_proj = nn.Linear(4, 4, bias=False)


class Block(nn.Module):
    def __init__(self):
        super().__init__()
        self.attn = Attention()
        self.cross_attn = Attention()


class Model(nn.Module):
    def __init__(self):
        super().__init__()
        self.transformer = nn.Module()
        self.transformer.h = nn.ModuleList([Block(), Block()])


def test_qkv_sharing_only_for_production_attention_names():
    # tests/test_optimizer.py:152-193 (selection part)
    matrices, _ = select_matrices(Model())
    src = {n: shared_source(n, matrices) for n in matrices}
    for i in (0, 1):
        q = f"transformer.h.{i}.attn.q_proj.weight"
        assert src[f"transformer.h.{i}.attn.k_proj.weight"] == q
        assert src[f"transformer.h.{i}.attn.v_proj.weight"] == q
        assert src[q] == q
        for p in ("q", "k", "v"):
            n = f"transformer.h.{i}.cross_attn.{p}_proj.weight"
            assert src[n] == n


def test_k_without_q_is_unshared():
    matrices, _ = select_matrices(Model(), lambda n, m: isinstance(m, nn.Linear) and "q_proj" not in n)
    assert shared_source("transformer.h.0.attn.k_proj.weight", matrices) == "transformer.h.0.attn.k_proj.weight"


def test_selection_default_and_filter():
    m = nn.Sequential(nn.Linear(4, 5), nn.Tanh(), nn.Linear(5, 2))
    mats, mods = select_matrices(m)
    assert list(mats) == ["0.weight", "2.weight"]
    frozen = nn.Sequential(nn.Linear(4, 5))
    frozen[0].weight.requires_grad_(False)
    with pytest.raises(ValueError, match="No eligible trainable linear weights found"):
        select_matrices(frozen)


def test_gpt_103m_layout():
    # BASELINE cfg4: 103,176,192 parameters; 54 selected matrices holding 63,700,992.
    with torch.device("meta"):
        model = GPT(GPT_103M)
    assert sum(p.numel() for p in model.parameters()) == 103_176_192
    mats, _ = select_matrices(model, transformer_filter)
    assert len(mats) == 54
    assert sum(p.numel() for p in mats.values()) == 63_700_992
    sources = {shared_source(n, mats) for n in mats}
    assert len(sources) == 36


def test_constructor_errors():
    with pytest.raises(ValueError, match="No eligible"):
        RankOneAWeightedPE(nn.Sequential(nn.Tanh()), 1e-3)
    # A bare module has no named submodule: nothing is selected (as in the
    # reference, whose selection skips the root module).
    with pytest.raises(ValueError, match="No eligible"):
        RankOneAWeightedPE(nn.Linear(4, 3), 1e-3)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        RankOneAWeightedPE(nn.Sequential(nn.Linear(4, 3)), 1e-3)  # CPU parameters: no fallback
    with pytest.raises(ValueError, match="s8_mode"):
        DiagonalWeightedPE(nn.Sequential(nn.Linear(4, 3)), 1e-3, s8_mode="fp16")
    # parameters on more than one device: refused before any is used
    with pytest.raises(ValueError, match="one device"):
        RankOneAWeightedPE(nn.Sequential(nn.Linear(4, 3), nn.Linear(3, 2, device="meta")), 1e-3)


def test_public_exports():
    assert S8_MARGIN == 1.35 and S8_MULTIPLIER == 1.0 and len(S8_COEFFICIENTS) == 5


def test_helper_factor_batching(monkeypatch):
    # The module-level rank-one helpers take factors with or without batch
    # dimensions and a 0-dim or batched coefficient (rank1_mapback is called
    # on 2-D values, tests/test_optimizer.py:46-54).
    from sandmuon_amd import optimizer as M
    monkeypatch.setattr(M, "_to_gpu", lambda t, dtype: torch.as_tensor(t).to(dtype).contiguous())
    vec, z, c = torch.rand(5), torch.rand(5), torch.tensor(-.4)
    for batch_shape in (torch.Size([]), torch.Size([3]), torch.Size([2, 3])):
        bv, bz, bc = M._batched_factor((vec, z, c), batch_shape, 5, torch.float64)
        n = max(1, batch_shape.numel())
        assert bv.shape == bz.shape == (n, 5) and bc.shape == (n,) and bc.dtype == torch.float64
    batched = (vec.expand(3, 5), z.expand(3, 5), c.expand(3))
    bv, _, bc = M._batched_factor(batched, torch.Size([3]), 5, torch.float32)
    assert bv.shape == (3, 5) and bc.shape == (3,)
    assert M._work_dtype(torch.zeros(2), torch.zeros(2, dtype=torch.float64)) == torch.float64
    assert M._work_dtype(torch.zeros(2, dtype=torch.bfloat16)) == torch.float32


def _bare_optimizer(params):
    """A DiagonalWeightedPE shell over CPU parameters: torch's Optimizer
    state without the GPU constructor (no hooks, no library calls), enough
    to run load_state_dict."""
    from sandmuon_amd import optimizer as M
    opt = M.DiagonalWeightedPE.__new__(M.DiagonalWeightedPE)
    torch.optim.Optimizer.__init__(opt, [dict(params=params[:1], use_muon=True),
                                         dict(params=params[1:], use_muon=False)], dict(lr=1e-3))
    return opt


def test_load_state_dict_keeps_float32_state_for_16bit_parameters():
    # torch casts floating state to the parameter dtype on load; the build
    # restores the saved float32 values (not their bf16 rounding).
    w = nn.Parameter(torch.zeros(3, 5, dtype=torch.bfloat16))
    b = nn.Parameter(torch.zeros(3, dtype=torch.bfloat16))
    opt = _bare_optimizer([w, b])
    g = torch.Generator().manual_seed(5)
    fine = lambda *shape: 1 + torch.rand(*shape, generator=g) * 2 ** -12  # not bf16-representable
    saved = {"state": {0: {"a_sum": fine(5), "a_first_sum": fine(5), "a_count": 0, "b_sum": fine(3),
                           "b_count": 0, "a_ema": fine(5), "a_mean_ema": fine(5), "b_ema": fine(3),
                           "momentum_buffer": fine(5, 3).t()},  # a transposed (non-contiguous) buffer
                       1: {"exp_avg": fine(3), "exp_avg_sq": fine(3), "step": 4}},
             "param_groups": [dict(opt.param_groups[0], params=[0]), dict(opt.param_groups[1], params=[1])]}
    opt.load_state_dict(saved)
    for i, p in enumerate((w, b)):
        for key, value in saved["state"][i].items():
            got = opt.state[p][key]
            if torch.is_tensor(value):
                assert got.dtype == torch.float32 and got.is_contiguous(), key
                assert torch.equal(got, value), key
                assert got.data_ptr() != value.data_ptr(), key  # a copy, not the caller's tensor
            else:
                assert got == value, key


def test_state_vectors_are_checked_before_launch():
    from sandmuon_amd.optimizer import _require_f32
    ok = torch.zeros(4)
    assert _require_f32(ok, 4, ok.device, "a_sum") is ok
    for bad in (torch.zeros(4, dtype=torch.bfloat16), torch.zeros(5), torch.zeros(8)[::2]):
        with pytest.raises(ValueError, match="contiguous float32"):
            _require_f32(bad, 4, ok.device, "a_sum")
