"""smx_matrix_step_static (the matrix step with its workspace in a static
device array, for callers that cannot allocate) against smx_matrix_step
with a caller workspace, both through the C ABI.

Bar: bit-identical parameters and momentum (the same kernels on the same
inputs), on two calls in a row on one GPU, the second with fewer and
smaller matrices, so that the second call runs over what the first left in
the shared array.  A set of matrices whose workspace exceeds the array is
refused before any launch."""
import pytest
import torch

from sandmuon_amd import _native

pytestmark = pytest.mark.gpu


def static_step():
    return _native.lib().smx_matrix_step_static


def make_inputs(device, shapes, seed, rank1):
    g = torch.Generator(device=device).manual_seed(seed)
    mats = []
    for rows, cols in shapes:
        m = dict(param=torch.randn(rows, cols, generator=g, device=device) * .02,
                 grad=torch.randn(rows, cols, generator=g, device=device) * 1e-3,
                 momentum=torch.randn(rows, cols, generator=g, device=device) * 1e-3,
                 inv_row=torch.rand(rows, generator=g, device=device) + .5,
                 inv_col=torch.rand(cols, generator=g, device=device) + .5)
        if rank1:
            m["z"] = torch.randn(cols, generator=g, device=device) * .3
            m["kappa"] = torch.full((1,), -.2, device=device)
        mats.append(m)
    return mats


def clone(mats):
    return [{k: v.clone() for k, v in m.items()} for m in mats]


def descs(mats):
    out = []
    for m in mats:
        d = _native.MatrixDesc(param=m["param"].data_ptr(), grad=m["grad"].data_ptr(),
                               momentum=m["momentum"].data_ptr(), inv_row=m["inv_row"].data_ptr(),
                               inv_col=m["inv_col"].data_ptr(), rows=m["param"].shape[0],
                               cols=m["param"].shape[1], lr=1e-2, momentum_beta=.8, grad_dtype=0, param_dtype=0)
        if "z" in m:
            d.z, d.kappa = m["z"].data_ptr(), m["kappa"].data_ptr()
        out.append(d)
    return (_native.MatrixDesc * len(out))(*out)


@pytest.mark.parametrize("rank1", [True, False])
@pytest.mark.parametrize("mode", ["comp_bf16", "fp32"])
def test_static_step_equals_workspace_step(device, mode, rank1):
    fn = static_step()
    code = _native.S8_MODES[mode]
    stream = _native.stream_of(device)
    calls = [[(768, 768)] * 3 + [(3072, 768)] * 2 + [(768, 3072)] * 2 + [(100, 300), (300, 100)],
             [(256, 384), (384, 256), (64, 64)]]
    for k, shapes in enumerate(calls):
        a = make_inputs(device, shapes, 100 + k, rank1)
        b = clone(a)
        need = _native.matrix_step_workspace_bytes(shapes, code)
        assert need <= 1 << 30  # SMX_MATRIX_STEP_STATIC_BYTES
        ws = torch.empty(need, dtype=torch.uint8, device=device)
        da, db = descs(a), descs(b)
        _native.matrix_step(list(da), code, ws)
        rc = fn(db, len(shapes), code, stream)
        assert rc == 0, _native.lib().smx_last_error()
        torch.cuda.synchronize()
        for i, (ma, mb) in enumerate(zip(a, b)):
            assert torch.equal(ma["param"], mb["param"]), (k, i, shapes[i])
            assert torch.equal(ma["momentum"], mb["momentum"]), (k, i, shapes[i])
            assert not torch.equal(ma["param"], make_inputs(device, shapes, 100 + k, rank1)[i]["param"])


def test_static_step_refuses_matrices_beyond_its_array(device):
    fn = static_step()
    # two 8192 x 8192 matrices need several GB of workspace; the call must
    # return before touching the (never dereferenced) pointers
    # The fake pointers are safe only while the size check refuses this set:
    # fail on the host if the workspace estimate ever fits the array.
    assert _native.matrix_step_workspace_bytes([(8192, 8192)] * 2, _native.S8_COMP_BF16) > 1 << 30
    d = _native.MatrixDesc(param=256, grad=256, momentum=256, inv_row=256, inv_col=256, rows=8192, cols=8192,
                           lr=1e-2, momentum_beta=.8)
    arr = (_native.MatrixDesc * 2)(d, d)
    assert fn(arr, 2, _native.S8_COMP_BF16, _native.stream_of(device)) == -5
    assert b"static scratch" in _native.lib().smx_last_error()
    assert fn(arr, 0, _native.S8_COMP_BF16, _native.stream_of(device)) == 0
