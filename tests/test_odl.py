"""The historical ODL plugin boundary on the host (no GPU): the registry
(reproduction/odl/optim/registry.py:21-75), the factory names and signature
(diagonal_weighted_pe.py:551-561), the historical matrix selection and its
errors (:178-220)."""
import pytest
from torch import nn

from sandmuon_amd import odl
from sandmuon_amd.workloads import GPT, GPT_TINY


class Attn(nn.Module):
    def __init__(self, with_q=True):
        super().__init__()
        if with_q:
            self.q_proj = nn.Linear(4, 4)
        self.k_proj = nn.Linear(4, 4)
        self.v_proj = nn.Linear(4, 4)


class Net(nn.Module):
    def __init__(self, with_q=True):
        super().__init__()
        self.transformer = nn.Module()
        blk = nn.Module()
        blk.attn = Attn(with_q)
        blk.mlp = nn.Linear(4, 8)
        self.transformer.h = nn.ModuleList([blk])
        self.lm_head = nn.Linear(4, 10)


def test_registered_names():
    assert odl.available_optimizers() == ["muon_raw_diagonal_weighted_pe", "sand_muon", "sand_muon_rank1"]


def test_unknown_name_lists_the_registry():
    with pytest.raises(ValueError) as e:
        odl.create_optimizer(Net(), optimizer_type="dense")
    assert str(e.value) == ("Unknown optimizer_type 'dense'. Available: "
                            "muon_raw_diagonal_weighted_pe, sand_muon, sand_muon_rank1")


def test_lookup_is_case_insensitive_and_passes_the_factory_signature():
    seen = {}

    @odl.register_optimizer("probe_opt")
    def _probe(model, *, lr, betas, weight_decay, device_type):
        seen.update(model=model, lr=lr, betas=betas, weight_decay=weight_decay, device_type=device_type)
        return "built"

    try:
        m = Net()
        assert odl.create_optimizer(m, optimizer_type="PROBE_OPT") == "built"
        assert seen == dict(model=m, lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1, device_type="cuda")
        odl.create_optimizer(m, lr=1e-2, betas=(.8, .9), weight_decay=0., optimizer_type="probe_opt",
                             device_type="cpu")
        assert seen["lr"] == 1e-2 and seen["betas"] == (.8, .9) and seen["device_type"] == "cpu"
    finally:
        del odl._REGISTRY["probe_opt"]


def test_historical_selection_is_transformer_blocks_only():
    from sandmuon_amd.optimizer import select_matrices
    names = list(select_matrices(Net(), odl.historical_filter)[0])
    assert names == ["transformer.h.0.attn.q_proj.weight", "transformer.h.0.attn.k_proj.weight",
                     "transformer.h.0.attn.v_proj.weight", "transformer.h.0.mlp.weight"]


def test_no_transformer_linear_is_a_value_error():
    with pytest.raises(ValueError, match=r"^No transformer\.h\.\* linear weights found$"):
        odl.DiagonalWeightedPE(nn.Sequential(nn.Linear(3, 3)), 1e-3)


def test_k_and_v_without_q_is_a_runtime_error():
    with pytest.raises(RuntimeError, match="^Split attention projection is missing q_proj$"):
        odl.RankOneAWeightedPE(Net(with_q=False), 1e-3)


@pytest.mark.parametrize("name", ["sand_muon", "SAND_MUON_RANK1", "muon_raw_diagonal_weighted_pe"])
def test_factories_reach_the_gpu_only_classes(name):
    # The selection passes; the build then refuses CPU parameters, as every
    # class of this package does (there is no CPU path).
    model = GPT(GPT_TINY)
    with pytest.raises(RuntimeError, match="ROCm GPU parameters only"):
        odl.create_optimizer(model, optimizer_type=name)
