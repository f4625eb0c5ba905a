"""HIP-graph replay of the UNet forward and of the denoise loop.

Every replay must equal the eager forward bit for bit: replays are checked
one by one with eager work and synchronisations between them, after the
input buffers are rewritten in place, and after the arguments change (a new
capture).  The denoise loop with graphs on equals the loop with graphs off.
"""
import pytest
import torch

from dollama_amd import unet as U
from oracle import unet_ref as OR

pytestmark = pytest.mark.gpu

TINY = U.UNetConfig(C0=64, C1=128, C2=192, depth1=1, depth2=2, cross_dim=96, text_dim=64, id_dim=16)


def _net():
    W = OR.random_weights(OR.TINY, seed=3)
    net = U.UNet(TINY)
    net.set_weights({k: v.half().cuda() for k, v in W.items()})
    net.prepare()
    return net


def _inputs(seed, B=2, H=32, W=32, L=77):
    g = torch.Generator().manual_seed(seed)
    lat = torch.randn(B, 4, H, W, generator=g).half().cuda()
    ehs = torch.randn(B, L, TINY.cross_dim, generator=g).half().cuda()
    text = torch.randn(B, TINY.text_dim, generator=g).half().cuda()
    ts = torch.tensor([999.0, 999.0][:B]).cuda()
    ids = torch.tensor([1024.0, 1024.0, 0.0, 0.0, 1024.0, 1024.0]).half().cuda()
    return lat, ts, ehs, text, ids


def test_forward_graph_replays_equal_eager(gpu):
    net = _net()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        lat, ts, ehs, text, ids = _inputs(1)
        out = torch.empty(2, 4, 32, 32, dtype=torch.float16, device="cuda")
        net.forward(lat, ts, ehs, text, ids, out=out)
        s.synchronize()
        ref = out.clone()
        net.set_graphs(True)
        for i in range(4):  # eager (first sight), capture + launch, then replays
            out.zero_()
            net.forward(lat, ts, ehs, text, ids, out=out)
            s.synchronize()
            assert torch.equal(out, ref), f"call {i} differs from the eager forward"
            junk = torch.randn(256, 256, device="cuda") @ torch.randn(256, 256, device="cuda")
            s.synchronize()
            del junk
        assert net.graphs_captured == 1
        # new values in the same buffers: the replay reads them
        lat2, ts2, ehs2, text2, _ = _inputs(2)
        lat.copy_(lat2)
        ehs.copy_(ehs2)
        text.copy_(text2)
        ts.fill_(500.0)
        net.forward(lat, ts, ehs, text, ids, out=out)
        s.synchronize()
        replay = out.clone()
        net.set_graphs(False)
        net.forward(lat, ts, ehs, text, ids, out=out)
        s.synchronize()
        assert torch.equal(replay, out), "replay on rewritten inputs differs from eager"
        # other arguments: captured separately, still exact
        net.set_graphs(True)
        out2 = torch.empty_like(out)
        for _ in range(3):
            net.forward(lat, ts, ehs, text, ids, out=out2)
            s.synchronize()
            assert torch.equal(out2, out)
        assert net.graphs_captured == 1  # set_graphs(False) dropped the first graph
    net.close()


def test_denoise_loop_with_graphs_equals_eager(gpu):
    net = _net()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        _, _, ehs, text, ids = _inputs(5)
        sig, _ = U.euler_schedule(5)
        g = torch.Generator().manual_seed(6)
        lat0 = (torch.randn(4, 32, 32, generator=g) * sig[0]).cuda()
        a = lat0.clone()
        U.denoise(net, a, ehs, text, ids, steps=5, guidance=6.0)
        s.synchronize()
        net.set_graphs(True)
        for i in range(3):
            b = lat0.clone()
            U.denoise(net, b, ehs, text, ids, steps=5, guidance=6.0)
            s.synchronize()
            assert torch.equal(a, b), f"denoise run {i} with graphs differs"
        assert net.graphs_captured == 1
    net.close()


def test_split_k_conv_captured_on_a_fresh_stream(gpu):
    """A conv whose heuristic picks split-K (2048 x 1280 x 11520: the
    1280-channel level's 3x3 conv at B=2), captured on a stream that never
    ran it eagerly: no workspace can be made under capture, so the captured
    launch runs unsplit; the capture succeeds, every replay gives the same
    bits, and they match the eager (split) result to fp32 summation order."""
    from dollama_amd import ops
    from tests._util import assert_close, randn, to_gpu
    print("[case] split-K conv 2048x1280x11520 captured on a fresh stream", flush=True)
    x = ops.nchw_to_nhwc(to_gpu(randn((2, 1280, 32, 32), 700)))
    wp = ops.pack_conv_weight(to_gpu(randn((1280, 1280, 3, 3), 701, std=0.01)))
    b = to_gpu(randn((1280,), 702, std=0.1))
    eager = ops.conv2d_nhwc(x, wp, KH=3, KW=3, bias=b)
    torch.cuda.synchronize()
    y = torch.empty_like(eager)
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            ops.conv2d_nhwc(x, wp, KH=3, KW=3, bias=b, out=y)
    outs = []
    for _ in range(3):
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        outs.append(y.clone())
    assert all(torch.equal(o, outs[0]) for o in outs), "replays differ"
    assert_close(outs[0], eager.float().cpu(), "captured unsplit vs eager split-K", rel_tol=1e-3,
                 cos_tol=0.999999)
