"""Statistics fused into the Linear's input cast and bias-gradient passes
(sandmuon_amd.fused) against the hook path and torch's own layer.

* smx_stats_cast: the low-precision copy equals torch's cast bit for bit and
  the slot rows equal smx_stats_accumulate's bit for bit;
* smx_stats_colsum: the slot rows equal smx_stats_accumulate's bit for bit;
  the column sums match an FP64 reference (rel. <= 1e-6);
* a fused nn.Linear under bf16 autocast gives torch's output, input gradient
  and weight gradient bit for bit, and the bias gradient within the bf16
  rounding torch's own bias gradient carries;
* smx_stats_gelu: the GELU equals torch's F.gelu bit for bit over every
  bf16 and f16 value, and its partials, added into slot rows, equal the
  slot rows smx_stats_accumulate leaves for its output bit for bit;
* smx_stats_relayout: the row-major copy of a head-transposed attention
  output equals torch's reshape bit for bit, and its partials, added into
  slot rows, equal the slot rows smx_stats_accumulate leaves for the copy
  bit for bit;
* a GPT step with fused statistics (with and without the GELU and the
  attention-output relayout fused) gives the hook path's statistics and
  matrix updates bit for bit.
"""
import copy

import pytest
import torch
from torch import nn

from sandmuon_amd import DiagonalWeightedPE, RankOneAWeightedPE, _native
from sandmuon_amd.fused import fuse_statistics
from sandmuon_amd.workloads import GPT, GPTConfig, transformer_filter

pytestmark = pytest.mark.gpu

SLOTS = 128


def fp64_colsum(x2d):
    return x2d.double().sum(0)


def rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-300)).item()


@pytest.mark.parametrize("rows,cols", [(16384, 768), (16384, 3072), (7, 5), (1000, 96), (33, 100)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("first", [True, False])
def test_stats_cast_matches_torch_cast_and_hook_slots(device, rows, cols, out_dtype, first):
    g = torch.Generator(device=device).manual_seed(rows + cols)
    x = torch.randn(rows, cols, generator=g, device=device) * 3 + 0.5
    ref_sq = torch.zeros(SLOTS, cols, device=device)
    ref_fs = torch.zeros(SLOTS, cols, device=device) if first else None
    _native.stats_accumulate(x, ref_sq, ref_fs)
    sq = torch.zeros(SLOTS, cols, device=device)
    fs = torch.zeros(SLOTS, cols, device=device) if first else None
    out = torch.empty(rows, cols, dtype=out_dtype, device=device)
    _native.stats_cast(x, sq, fs, out)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), x.to(out_dtype).view(torch.int16))
    assert torch.equal(sq, ref_sq)
    if first:
        assert torch.equal(fs, ref_fs)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_stats_gelu_equals_torch_gelu_on_every_value(device, dtype):
    h = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16).view(dtype).reshape(256, 256).to(device)
    out = torch.empty_like(h)
    chunks = _native.stats_slot_rows(256, SLOTS)
    part = torch.empty(chunks, 256, device=device)
    _native.stats_gelu(h, out, part, None, SLOTS)
    want = torch.nn.functional.gelu(h)
    torch.cuda.synchronize()
    nan = torch.isnan(want)
    assert torch.equal(torch.isnan(out), nan)
    assert torch.equal(out[~nan].view(torch.int16), want[~nan].view(torch.int16))


@pytest.mark.parametrize("rows,cols", [(16384, 3072), (16384 * 3 + 5, 768), (513, 8), (1, 16), (3, 1024)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("first", [True, False])
def test_stats_gelu_partials_equal_hook_slots_of_its_output(device, rows, cols, dtype, first):
    g = torch.Generator(device=device).manual_seed(rows + 3 * cols)
    h = (torch.randn(rows, cols, generator=g, device=device) * 2).to(dtype)
    # slot rows that already hold sums of earlier calls
    base_sq = torch.rand(SLOTS, cols, generator=g, device=device)
    base_fs = torch.randn(SLOTS, cols, generator=g, device=device) if first else None
    ref_sq = base_sq.clone()
    ref_fs = base_fs.clone() if first else None
    _native.stats_accumulate(torch.nn.functional.gelu(h), ref_sq, ref_fs)
    out = torch.empty_like(h)
    chunks = _native.stats_slot_rows(rows, SLOTS)
    part_sq = torch.empty(chunks, cols, device=device)
    part_fs = torch.empty(chunks, cols, device=device) if first else None
    _native.stats_gelu(h, out, part_sq, part_fs, SLOTS)
    sq, fs = base_sq.clone(), base_fs.clone() if first else None
    _native.stats_add_partials(sq, part_sq, fs, part_fs)
    torch.cuda.synchronize()
    # equal values: torch's own small-tensor path can give +0 where its
    # vectorised path (and this kernel) give -0 for an underflowing negative
    assert torch.equal(out, torch.nn.functional.gelu(h))
    assert torch.equal(sq, ref_sq)
    if first:
        assert torch.equal(fs, ref_fs)


def test_stats_gelu_refuses_unaligned_widths(device):
    h = torch.randn(4, 12, device=device).to(torch.bfloat16)
    with pytest.raises(ValueError, match="multiples of 8"):
        _native.stats_gelu(h, torch.empty_like(h), torch.empty(1, 12, device=device), None, SLOTS)


@pytest.mark.parametrize("b,h,t,d,pad", [(2, 12, 1024, 64, 0), (1, 16, 512, 128, 0), (4, 3, 512, 8, 0),
                                         (2, 5, 1536, 24, 0), (2, 4, 1024, 64, 32)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("first", [True, False])
def test_stats_relayout_copy_and_partials_equal_reshape_and_hook_slots(device, b, h, t, d, pad, dtype, first):
    g = torch.Generator(device=device).manual_seed(b * h * t + d)
    # [batch, heads, seq, head_dim] as attention returns it (pad: a view of
    # a wider buffer, so the seq stride is not head_dim)
    full = (torch.randn(b, h, t, d + pad, generator=g, device=device) * 3 - 0.25).to(dtype)
    y = full[..., :d].transpose(1, 2)          # [batch, seq, heads, head_dim], not contiguous
    want = y.reshape(b * t, h * d)
    cols = h * d
    base_sq = torch.rand(SLOTS, cols, generator=g, device=device)
    base_fs = torch.randn(SLOTS, cols, generator=g, device=device) if first else None
    ref_sq = base_sq.clone()
    ref_fs = base_fs.clone() if first else None
    _native.stats_accumulate(want, ref_sq, ref_fs)
    out = torch.empty(b * t, cols, dtype=dtype, device=device)
    chunks = _native.stats_slot_rows(b * t, SLOTS)
    part_sq = torch.empty(chunks, cols, device=device)
    part_fs = torch.empty(chunks, cols, device=device) if first else None
    _native.stats_relayout(y, out, part_sq, part_fs, SLOTS)
    sq, fs = base_sq.clone(), base_fs.clone() if first else None
    _native.stats_add_partials(sq, part_sq, fs, part_fs)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))
    assert torch.equal(sq, ref_sq)
    if first:
        assert torch.equal(fs, ref_fs)


def test_stats_relayout_refuses_chunks_across_sequences(device):
    y = torch.randn(2, 4, 768, 64, device=device).to(torch.bfloat16).transpose(1, 2)
    out = torch.empty(2 * 768, 256, dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError, match="multiple of the row chunk"):
        _native.stats_relayout(y, out, torch.empty(3, 256, device=device), None, SLOTS)


def test_stats_cast_strided_rows(device):
    base = torch.randn(300, 130, device=device)
    x = base[:, :128]  # row stride 130
    out_base = torch.empty(300, 136, dtype=torch.bfloat16, device=device)
    out = out_base[:, :128]
    sq, ref = torch.zeros(SLOTS, 128, device=device), torch.zeros(SLOTS, 128, device=device)
    _native.stats_cast(x, sq, None, out)
    _native.stats_accumulate(x, ref, None)
    torch.cuda.synchronize()
    assert torch.equal(out, x.to(torch.bfloat16)) and torch.equal(sq, ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("rows,cols", [(16384, 768), (16384, 3072), (0, 64), (1, 16), (130, 100), (33, 7)])
def test_stats_colsum_matches_fp64_and_hook_slots(device, dtype, rows, cols):
    g = torch.Generator(device=device).manual_seed(7 * rows + cols)
    x = (torch.randn(rows, cols, generator=g, device=device) * 1e-3 + 2e-4).to(dtype)
    ws = torch.full((_native.stats_colsum_workspace_bytes(cols, SLOTS),), 255, dtype=torch.uint8, device=device)
    sq, ref = torch.zeros(SLOTS, cols, device=device), torch.zeros(SLOTS, cols, device=device)
    colsum = torch.full((cols,), float("nan"), device=device)
    for rep in range(2):  # the workspace starts as garbage (NaN bytes) and is reused
        _native.stats_colsum(x, sq, colsum, ws)
        if rows:
            _native.stats_accumulate(x, ref, None)
        torch.cuda.synchronize()
        assert torch.equal(sq, ref), rep
        want = fp64_colsum(x)
        if rows == 0:
            assert torch.equal(colsum, torch.zeros(cols, device=device))
        else:
            assert rel(colsum, want) <= 1e-6, rep
            # elementwise: within FP32 rounding of the magnitudes summed
            bound = 1e-6 * x.double().abs().sum(0) + 1e-30
            assert ((colsum.double() - want).abs() <= bound).all()


def _native_linear(lin, x, dy):
    lin = copy.deepcopy(lin)
    x = x.detach().clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = lin(x)
    y.backward(dy)
    return y.detach(), x.grad, lin.weight.grad, None if lin.bias is None else lin.bias.grad


@pytest.mark.parametrize("bias", [True, False])
@pytest.mark.parametrize("in_dtype", [torch.float32, torch.bfloat16])
def test_fused_linear_matches_autocast_linear(device, bias, in_dtype):
    torch.manual_seed(5)

    class Net(nn.Module):
        def __init__(self):
            super().__init__()
            self.fc = nn.Linear(768, 3072, bias=bias)

    net = Net().to(device)
    ref_fc = copy.deepcopy(net.fc)
    opt = RankOneAWeightedPE(net, 1e-2)
    handle = fuse_statistics(opt)
    assert handle.fused_names == ["fc.weight"] and opt.handles == []
    x = (torch.randn(4, 1024, 768, device=device) + 0.3).to(in_dtype)
    dy = (torch.randn(4, 1024, 3072, device=device) * 1e-3).bfloat16()
    ry, rdx, rdw, rdb = _native_linear(ref_fc, x, dy)
    xx = x.detach().clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = net.fc(xx)
    y.backward(dy)
    torch.cuda.synchronize()
    assert y.dtype == ry.dtype and torch.equal(y, ry)
    assert xx.grad.dtype == rdx.dtype and torch.equal(xx.grad, rdx)
    assert torch.equal(net.fc.weight.grad, rdw)
    if bias:
        want = fp64_colsum(dy.reshape(-1, 3072).float())
        assert net.fc.bias.grad.dtype == torch.float32
        assert rel(net.fc.bias.grad, want) <= 1e-6
        # torch's bias gradient is the bf16-rounded sum
        assert ((net.fc.bias.grad - rdb).abs() <= rdb.abs() * 2 ** -8 + 1e-6).all()
    # the statistics are the hooks' own
    st = opt.state[net.fc.weight]
    assert st["a_count"] == st["b_count"] == 4096
    handle.close()
    assert len(opt.handles) == 1 and "forward" not in net.fc.__dict__
    opt.close()


def test_qkv_share_the_source_cast_of_an_unmodified_input(device):
    class Attn(nn.Module):
        def __init__(self):
            super().__init__()
            self.q_proj, self.k_proj, self.v_proj = nn.Linear(64, 64), nn.Linear(64, 64), nn.Linear(64, 64)

    class Net(nn.Module):  # the q/k/v sharing applies to transformer.h.N.attn.*
        def __init__(self):
            super().__init__()
            self.transformer = nn.Module()
            blk = nn.Module()
            blk.attn = Attn()
            self.transformer.h = nn.ModuleList([blk])

    net = Net().to(device)
    opt = RankOneAWeightedPE(net, 1e-2)
    fuse_statistics(opt)
    x = torch.randn(2, 16, 64, device=device, requires_grad=True)
    a = net.transformer.h[0].attn
    with torch.autocast("cuda", dtype=torch.bfloat16):
        yq, yk, yv = a.q_proj(x), a.k_proj(x), a.v_proj(x)
    saved = [y.grad_fn.saved_tensors[0] for y in (yq, yk, yv)]
    assert saved[0].data_ptr() == saved[1].data_ptr() == saved[2].data_ptr()
    assert torch.equal(saved[0], x.detach().to(torch.bfloat16))
    # an input modified in place after the source's cast is cast again
    with torch.autocast("cuda", dtype=torch.bfloat16):
        x2 = x.detach().clone()
        yq = a.q_proj(x2)
        x2.mul_(2)
        yk = a.k_proj(x2)
    assert yk.grad_fn.saved_tensors[0].data_ptr() != yq.grad_fn.saved_tensors[0].data_ptr()
    assert torch.equal(yk.grad_fn.saved_tensors[0], x2.to(torch.bfloat16))
    opt.close()


def _gpt_pair(device, cfg, seed, opt_cls):
    model = GPT(cfg)
    model.init_weights(seed)
    model = model.to(device)
    twin = copy.deepcopy(model)
    a = opt_cls(model, 1e-2, module_filter=transformer_filter)
    b = opt_cls(twin, 1e-2, module_filter=transformer_filter)
    return model, twin, a, b


@pytest.mark.parametrize("opt_cls,amp", [(RankOneAWeightedPE, torch.bfloat16), (DiagonalWeightedPE, torch.bfloat16),
                                         (RankOneAWeightedPE, torch.float16)])
@pytest.mark.parametrize("gelu", [False, True], ids=["linears", "linears_and_gelu"])
def test_fused_gpt_step_equals_hook_step(device, opt_cls, amp, gelu):
    cfg = GPTConfig(vocab=257, ctx=128, layers=2, width=256, heads=4, mlp=1024)
    model, twin, hooked, fused_opt = _gpt_pair(device, cfg, 11, opt_cls)
    handle = fuse_statistics(fused_opt, twin if gelu else None)
    assert len(handle.fused_names) == 12 and fused_opt.handles == []
    g = torch.Generator().manual_seed(12)
    gm, gt = dict(model.named_parameters()), dict(twin.named_parameters())
    # Test-only tensor hooks on the fused layers' outputs record the
    # cotangents (the fused layers themselves use no hooks).
    captured = {}
    for name in handle.fused_names:
        module = dict(twin.named_modules())[name[: -len(".weight")]]
        store = captured.setdefault(name[: -len("weight")] + "bias", [])

        def fwd_hook(mod, inputs, output, store=store):
            output.register_hook(lambda grad: store.append(grad.detach().clone()))
        module.register_forward_hook(fwd_hook)
    for step in range(2):
        # The biases take slightly different AdamW steps (their gradients
        # differ in rounding); start every step from the same parameters.
        with torch.no_grad():
            for n, p in gm.items():
                gt[n].copy_(p)
        for opt in (hooked, fused_opt):
            opt.zero_grad(set_to_none=True)
        for mb in range(3):
            idx = torch.randint(0, cfg.vocab, (4, cfg.ctx), generator=g).to(device)
            tgt = torch.randint(0, cfg.vocab, (4, cfg.ctx), generator=g).to(device)
            for m in (model, twin):
                with torch.autocast("cuda", dtype=amp):
                    loss = m(idx, tgt) / 3
                loss.backward()
        for n in hooked.named_matrices:
            assert torch.equal(gm[n].grad, gt[n].grad), n
        # every MLP's GELU ran fused and its output's statistic was taken by
        # the MLP's c_proj
        assert handle.gelu_calls == handle.gelu_taken == (3 * cfg.layers * (step + 1) if gelu else 0)
        # Linear biases: the fused gradient is the FP32 column sum of the
        # captured cotangents, torch's the bf16-rounded one.  Both are held
        # against the FP64 sum: the fused one within FP32 rounding of the
        # magnitudes summed, and never further from it than torch's.
        for name, deltas in captured.items():
            d = torch.cat([t.reshape(-1, t.shape[-1]) for t in deltas]).double()
            want, mag = d.sum(0), d.abs().sum(0)
            err_fused = (gt[name].grad.double() - want).abs()
            err_torch = (gm[name].grad.double() - want).abs()
            assert (err_fused <= 1e-6 * mag + 1e-30).all(), name
            assert err_fused.max() <= err_torch.max(), name
            deltas.clear()
        hooked.step()
        fused_opt.step()
        torch.cuda.synchronize()
        for n, p in hooked.named_matrices.items():
            q = fused_opt.named_matrices[n]
            sa, sb = hooked.state[p], fused_opt.state[q]
            for key in ("a_ema", "a_mean_ema", "b_ema"):
                if key in sa:
                    assert torch.equal(sa[key], sb[key]), (step, n, key)
            assert torch.equal(p, q), (step, n)
    handle.close()
    assert len(fused_opt.handles) == 12
    hooked.close()
    fused_opt.close()


class _HeadsMajor(nn.Module):
    """A projection pair around a heads-major activation, as a manual
    attention (softmax(Q K^T) V) or any per-head op leaves it: the input of
    c_proj is the relayout copy of a [batch, heads, seq, head_dim] tensor
    (SDPA on this stack already returns its output seq-major, so the GPT's
    reshape is a view with no copy to fuse into)."""

    def __init__(self, width=256, heads=4):
        super().__init__()
        self.heads = heads
        self.q_proj = nn.Linear(width, width)
        self.c_proj = nn.Linear(width, width)

    def forward(self, x):
        b, t, c = x.shape
        h = self.q_proj(x).view(b, t, self.heads, c // self.heads).transpose(1, 2).contiguous()
        h = torch.nn.functional.silu(h) * 1.5
        return self.c_proj(h.transpose(1, 2).reshape(b, t, c))


@pytest.mark.parametrize("opt_cls,amp", [(RankOneAWeightedPE, torch.bfloat16), (DiagonalWeightedPE, torch.float16)])
def test_fused_relayout_step_equals_hook_step(device, opt_cls, amp):
    torch.manual_seed(3)
    model = _HeadsMajor().to(device)
    twin = copy.deepcopy(model)
    hooked, fused_opt = opt_cls(model, 1e-2), opt_cls(twin, 1e-2)
    with pytest.raises(ValueError, match="unknown activations"):
        fuse_statistics(fused_opt, twin, activations=("gelu", "softmax"))
    handle = fuse_statistics(fused_opt, twin, activations=("relayout",))
    g = torch.Generator(device=device).manual_seed(4)
    for step in range(2):
        for opt in (hooked, fused_opt):
            opt.zero_grad(set_to_none=True)
        for mb in range(3):
            x = torch.randn(2, 512, 256, generator=g, device=device)
            for m in (model, twin):
                with torch.autocast("cuda", dtype=amp):
                    loss = m(x).float().square().mean() / 3
                loss.backward()
        assert handle.relayout_calls == handle.relayout_taken == 3 * (step + 1)
        assert handle.gelu_calls == 0
        hooked.step()
        fused_opt.step()
        torch.cuda.synchronize()
        for n, p in hooked.named_matrices.items():
            q = fused_opt.named_matrices[n]
            for key in ("a_ema", "a_mean_ema", "b_ema"):
                if key in hooked.state[p]:
                    assert torch.equal(hooked.state[p][key], fused_opt.state[q][key]), (step, n, key)
            assert torch.equal(p, q), (step, n)
    # a sequence that is not a multiple of the 512-row chunk keeps the
    # separate read (the copy is torch's)
    with torch.autocast("cuda", dtype=amp):
        twin(torch.randn(2, 384, 256, device=device)).float().sum().backward()
    assert handle.relayout_calls == 6
    handle.close()
    hooked.close()
    fused_opt.close()


class _HeadSlice(nn.Module):
    """A reshape that is a view in torch (a head slice of a packed qkv with
    stride(h) == head_dim, flattened back)."""

    def __init__(self, width=256, heads=4):
        super().__init__()
        self.heads = heads
        self.qkv = nn.Linear(width, 3 * width)
        self.c_proj = nn.Linear(width, width)
        self.seen = []

    def forward(self, x):
        b, t, c = x.shape
        qkv = self.qkv(x).view(b, t, 3 * self.heads, c // self.heads)
        q = qkv[:, :, : self.heads]          # non-contiguous, stride(2) == head_dim
        flat = q.reshape(b, t, c)            # torch: a view of qkv
        self.seen.append((flat._base is not None, flat.data_ptr() == q.data_ptr()))
        return self.c_proj(flat)


def test_fused_relayout_keeps_reshape_views(device):
    torch.manual_seed(5)
    model = _HeadSlice().to(device)
    opt = RankOneAWeightedPE(model, 1e-2)
    handle = fuse_statistics(opt, model, activations=("relayout",))
    x = torch.randn(2, 512, 256, device=device)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        model(x).float().square().mean().backward()
    assert model.seen == [(True, True)]  # still a view of the same storage
    assert handle.relayout_calls == 0
    handle.close()
    opt.close()
