"""The allocation-free routed stack decode against the workspace entry point
it varies (aima_moe_stack_decode_routed), through the C ABI: same kernels, so
the routes must be identical and the outputs bit-identical; two calls in a
row, the second on a smaller input (fewer layers, smaller k), so that the
shared scratch array's leftover contents from the first call cannot leak
into the second."""

import ctypes as C

import pytest
import torch

pytestmark = pytest.mark.gpu


def _routed(pkg, layers, routers, x, k, noalloc):
    L = pkg._lib
    n = len(layers)
    arr = pkg.ops._layers_c(layers)
    rt = (L.U4TensorC * n)(*[r.c() for r in routers])
    dev = x.device
    ids = torch.full((n, k), -1, dtype=torch.int32, device=dev)
    w = torch.zeros((n, k), dtype=torch.float32, device=dev)
    out = torch.empty(layers[0].hidden, dtype=torch.float16, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        err = torch.zeros(1, dtype=torch.int32, device=dev)
        L.call("aima_moe_stack_decode_routed_noalloc", arr, rt, n, 1e-6, x.data_ptr(), k,
               pkg.MIN_WEIGHT_SUM, ids.data_ptr(), w.data_ptr(), out.data_ptr(), err.data_ptr(),
               stream)
        torch.cuda.synchronize()
        assert int(err.item()) == 0
    else:
        ws = pkg.Workspace(dev)
        buf = ws.get(L.size_query("aima_moe_decode_workspace_size", C.byref(arr[0]), k))
        L.call("aima_moe_stack_decode_routed", arr, rt, n, 1e-6, x.data_ptr(), k,
               pkg.MIN_WEIGHT_SUM, ids.data_ptr(), w.data_ptr(), out.data_ptr(), buf.data_ptr(),
               buf.numel(), stream)
        torch.cuda.synchronize()
        ws.check()
    return out, ids, w


def test_noalloc_matches_workspace_entry(pkg, dev):
    layers = [pkg.synth.moe_layer(2048, 512, 256, 128, seed=700 + l, device=dev)
              for l in range(4)]
    routers = [pkg.synth.u4_weight(1, 256, 2048, 128, pkg.synth.generator(710 + l, dev), dev)
               for l in range(4)]
    x = pkg.synth.activations(1, 2048, 720, dev)[0].contiguous()
    x2 = pkg.synth.activations(1, 2048, 721, dev)[0].contiguous()
    # first call: 4 layers, k = 8; second: 2 layers, k = 4 on another input
    for n, k, inp in ((4, 8, x), (2, 4, x2)):
        a = _routed(pkg, layers[:n], routers[:n], inp, k, noalloc=False)
        b = _routed(pkg, layers[:n], routers[:n], inp, k, noalloc=True)
        assert torch.equal(a[1], b[1]), f"routes differ (n={n}, k={k})"
        assert torch.equal(a[2], b[2])
        assert torch.equal(a[0], b[0]), f"outputs differ (n={n}, k={k})"
        assert (b[1] >= 0).all()


def test_noalloc_graph_capture_replays(pkg, dev):
    """The use the entry point is for: code under HIP graph capture.  One
    eager call first (it resolves the scratch array's address for this
    device, which the entry point does once per device and which is not
    meant to run under capture), then the call is captured once and
    replayed three times, with an eager call on another input in between
    (it overwrites the shared scratch array): every replay equals the eager
    result bit for bit, routes included."""
    L = pkg._lib
    n, k = 2, 8
    layers = [pkg.synth.moe_layer(2048, 512, 64, 128, seed=760 + l, device=dev)
              for l in range(n)]
    routers = [pkg.synth.u4_weight(1, 64, 2048, 128, pkg.synth.generator(770 + l, dev), dev)
               for l in range(n)]
    x = pkg.synth.activations(1, 2048, 780, dev)[0].contiguous()
    other = pkg.synth.activations(1, 2048, 781, dev)[0].contiguous()
    ref = _routed(pkg, layers, routers, x, k, noalloc=True)
    arr = pkg.ops._layers_c(layers)
    rt = (L.U4TensorC * n)(*[r.c() for r in routers])
    ids = torch.full((n, k), -1, dtype=torch.int32, device=dev)
    w = torch.zeros((n, k), dtype=torch.float32, device=dev)
    out = torch.empty(2048, dtype=torch.float16, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)

    def call():
        L.call("aima_moe_stack_decode_routed_noalloc", arr, rt, n, 1e-6, x.data_ptr(), k,
               pkg.MIN_WEIGHT_SUM, ids.data_ptr(), w.data_ptr(), out.data_ptr(),
               err.data_ptr(), torch.cuda.current_stream().cuda_stream)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    for _ in range(3):
        out.zero_()
        ids.fill_(-1)
        w.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert int(err.item()) == 0
        assert torch.equal(out, ref[0])
        assert torch.equal(ids, ref[1])
        assert torch.equal(w, ref[2])
        _routed(pkg, layers, routers, other, k, noalloc=True)  # eager work in between
