"""novaq_conv2d_backward_noalloc (the allocation-free Conv2d backward, its
workspace a static device array) against novaq_conv2d_backward with a
caller-allocated workspace, through the C ABI: the same kernels, so all three
gradients are bit-identical, on three calls in a row (the second smaller, so it
runs over what the first left in the shared scratch; the third with one input
channel, whose sums and grad_input share one launch), and a request beyond
the scratch's 32 MiB is refused with NOVAQ_ESCRATCH before any launch."""
import numpy as np
import pytest
import torch

import oracle as O
from novann_amd import _lib
from tests.gpu_util import to_dev

pytestmark = pytest.mark.gpu


def grads(noalloc, g, x, wq, s, geo):
    N, C, H, W, Co, K, st, pd, mode = geo
    OH, OW = (H + 2 * pd - K) // st + 1, (W + 2 * pd - K) // st + 1
    assert g.shape == (N, Co, OH, OW)
    lib = _lib.load()
    gi = torch.full((N, C, H, W), np.nan, device="cuda")
    gw = torch.full((Co, C, K, K), np.nan, device="cuda")
    gb = torch.full((Co,), np.nan, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    common = (g.data_ptr(), x.data_ptr(), N, C, H, W, wq.data_ptr(), _lib.E2M1, s.data_ptr(), Co,
              K, K, st, st, pd, pd, _lib.PAD_MODES[mode], gi.data_ptr(), gw.data_ptr(),
              gb.data_ptr())
    if noalloc:
        rc = lib.novaq_conv2d_backward_noalloc(*common, stream)
        ws = None
    else:
        nb = lib.novaq_conv2d_backward_workspace(N, C, Co, K, K, _lib.E2M1)
        ws = torch.empty(nb, dtype=torch.uint8, device="cuda")
        rc = lib.novaq_conv2d_backward(*common, ws.data_ptr(), nb, stream)
    assert rc == _lib.OK, rc
    torch.cuda.synchronize()
    del ws
    return [t.cpu().numpy() for t in (gi, gw, gb)]


def inputs(geo, seed):
    N, C, H, W, Co, K, st, pd, mode = geo
    OH, OW = (H + 2 * pd - K) // st + 1, (W + 2 * pd - K) // st + 1
    rng = np.random.default_rng(seed)
    x = torch.from_numpy(rng.uniform(0, 1, (N, C, H, W)).astype(np.float32)).cuda()
    g = torch.from_numpy(rng.standard_normal((N, Co, OH, OW)).astype(np.float32)).cuda()
    w = (rng.standard_normal((Co, C, K, K)) * np.sqrt(2.0 / (C * K * K))).astype(np.float32)
    s = O.scale_from_amax(O.amax(w), O.E2M1)
    wq = to_dev(O.cast(w.reshape(-1), O.F32, O.E2M1, scale=s), O.E2M1)
    return g, x, wq, torch.tensor([s], dtype=torch.float32, device="cuda")


# config [5]'s conv2 at batch 256 (30.8 MB of the 32 MiB scratch), then a
# smaller, differently shaped call (stride 2, reflect: the general kernels),
# then config [5]'s conv1 (one input channel: the one-input-channel kernels)
CALLS = [(256, 32, 28, 28, 64, 3, 1, 1, "zeros"), (3, 5, 11, 9, 7, 3, 2, 1, "reflect"),
         (256, 1, 28, 28, 32, 3, 1, 1, "zeros")]


def test_noalloc_matches_workspace_entry_point_twice():
    lib = _lib.load()
    for i, geo in enumerate(CALLS):
        N, C, H, W, Co, K = geo[:6]
        need = lib.novaq_conv2d_backward_workspace(N, C, Co, K, K, _lib.E2M1)
        print(f"noalloc call {i}: {geo}, workspace {need} B", flush=True)
        assert 0 < need <= 32 << 20
        args = inputs(geo, seed=i)
        got = grads(True, *args, geo)
        want = grads(False, *args, geo)
        for a, b in zip(got, want):
            assert not np.isnan(a).any()
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_noalloc_refuses_requests_beyond_the_scratch():
    lib = _lib.load()
    # C_out x C*KH*KW fp32 partials per chunk: 512 x 512 x 9 x 4 B x chunks > 32 MiB
    N, C, H, W, Co, K = 64, 512, 8, 8, 512, 3
    assert lib.novaq_conv2d_backward_workspace(N, C, Co, K, K, _lib.E2M1) > 32 << 20
    # real buffers of the call's sizes (zeros), so that a regression that
    # launched before the size check would compute garbage, not fault
    x = torch.zeros((N, C, H, W), device="cuda")
    g = torch.zeros((N, Co, H, W), device="cuda")
    wq = torch.zeros(Co * C * K * K // 2, dtype=torch.uint8, device="cuda")
    gi = torch.full((N, C, H, W), np.nan, device="cuda")
    gw = torch.full((Co, C, K, K), np.nan, device="cuda")
    gb = torch.full((Co,), np.nan, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.novaq_conv2d_backward_noalloc(g.data_ptr(), x.data_ptr(), N, C, H, W, wq.data_ptr(),
                                           _lib.E2M1, None, Co, K, K, 1, 1, 1, 1, 0,
                                           gi.data_ptr(), gw.data_ptr(), gb.data_ptr(), stream)
    torch.cuda.synchronize()
    assert rc == _lib.ESCRATCH
    assert b"scratch" in lib.novaq_status_string(_lib.ESCRATCH)
    # refused before any launch: the outputs are untouched
    assert torch.isnan(gw).all() and torch.isnan(gb).all() and torch.isnan(gi).all()
