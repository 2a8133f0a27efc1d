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

