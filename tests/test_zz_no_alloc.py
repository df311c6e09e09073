"""`qqt_l1_grad_noalloc` (the first-layer weight gradient with its chunk
partials in the library's static device scratch instead of a caller
workspace) against `qqt_l1_grad` through the C ABI (needs an MI355X).

Two calls in a row on the same GPU, the second with a smaller batch (so it
reads scratch the first call left behind only where it wrote it itself),
then a strided observation buffer: each result must equal `qqt_l1_grad`'s
on the same inputs bit for bit (same plan, same kernels).  An observation
wider than the scratch's maximum is rejected before any launch."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

K0 = 2366


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _inputs(b, seed, dev, stride=K0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.rand((b, stride), generator=g) < 0.2).float()
    x = x * torch.where(torch.rand((b, stride), generator=g) < 0.7, torch.ones(1),
                        torch.rand((b, stride), generator=g))
    dz1 = torch.randn((b, 128), generator=g) * 0.01
    amax = float(dz1.abs().max())
    import math
    scale = torch.tensor([2.0 ** (14 - math.ceil(math.log2(amax)))])
    return x.half().to(dev), dz1.to(dev), scale.to(dev)


def _args(x16, dz1, scale, out, k0=K0):
    from qqtsim import _capi

    a = _capi.L1GradArgsC()
    a.batch, a.k0, a.obs_stride = x16.shape[0], k0, x16.stride(0)
    a.obs, a.dz1, a.dz_scale, a.dw0 = x16.data_ptr(), dz1.data_ptr(), scale.data_ptr(), \
        out.data_ptr()
    return a


def _with_workspace(dev, x16, dz1, scale):
    from qqtsim import _capi

    lib = _capi.lib()
    out = torch.full((128, K0), float("nan"), dtype=torch.float32, device=dev)
    a = _args(x16, dz1, scale, out)
    need = lib.qqt_l1_grad_workspace_floats(x16.shape[0], K0)
    ws = torch.empty(need, dtype=torch.float32, device=dev)
    a.workspace, a.workspace_floats = ws.data_ptr(), need
    _capi.check(lib.qqt_l1_grad(a, _capi.stream_handle(dev)))
    torch.cuda.synchronize()
    return out


def _no_alloc(dev, x16, dz1, scale):
    from qqtsim import _capi

    out = torch.full((128, K0), float("nan"), dtype=torch.float32, device=dev)
    a = _args(x16, dz1, scale, out)          # workspace left NULL: the call must not need it
    _capi.check(_capi.lib().qqt_l1_grad_noalloc(a, _capi.stream_handle(dev)))
    torch.cuda.synchronize()
    return out


def test_no_alloc_equals_workspace_entry_point(dev):
    for b, seed in ((180_224, 1), (3_001, 2), (1, 3)):
        print(f"[no_alloc] batch {b}", flush=True)
        x16, dz1, scale = _inputs(b, seed, dev)
        want = _with_workspace(dev, x16, dz1, scale)
        got = _no_alloc(dev, x16, dz1, scale)
        assert torch.isfinite(got).all(), b
        assert torch.equal(got, want), b


def test_no_alloc_strided_observation(dev):
    x16, dz1, scale = _inputs(5_000, 4, dev, stride=K0 + 6)
    assert torch.equal(_no_alloc(dev, x16, dz1, scale), _with_workspace(dev, x16, dz1, scale))


def test_no_alloc_rejects_wider_observation(dev):
    from qqtsim import _capi

    lib = _capi.lib()
    x16 = torch.zeros((64, 2562), dtype=torch.float16, device=dev)
    dz1 = torch.zeros((64, 128), dtype=torch.float32, device=dev)
    out = torch.zeros((128, 2562), dtype=torch.float32, device=dev)
    a = _args(x16, dz1, torch.ones(1, device=dev), out, k0=2562)
    with pytest.raises(ValueError, match="exceeds the static scratch"):
        _capi.check(lib.qqt_l1_grad_noalloc(a, _capi.stream_handle(dev)))
