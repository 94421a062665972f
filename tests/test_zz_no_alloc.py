"""batteries_tensor_product_backward_l3_noalloc: the weighted backward with its
grad_W partials in the library's static device scratch instead of a caller
workspace.  Called through the C ABI and checked bit-exactly against
batteries_tensor_product_backward_l3 on the same inputs (the two share every
kernel), on two calls in a row, the second smaller, plus the size limit."""
import ctypes
import os

import numpy as np
import pytest
import torch

from helpers import gen, normwise_err, unit_vectors
from oracle import tp as otp

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(REPO, "batmobile-evo_amd", "lib", "libbatmobile_hip.so")
SCRATCH_BYTES = 24 << 20
ERR_SCRATCH = -4

P = ctypes.c_void_p


def _lib():
    lib = ctypes.CDLL(LIB)
    lib.batteries_tensor_product_backward_workspace_bytes.restype = ctypes.c_size_t
    lib.batteries_tensor_product_backward_workspace_bytes.argtypes = [ctypes.c_int64, ctypes.c_int,
                                                                      ctypes.c_int]
    lib.batteries_tensor_product_backward_l3.restype = ctypes.c_int
    lib.batteries_tensor_product_backward_l3.argtypes = [P] * 7 + [ctypes.c_int64, ctypes.c_int,
                                                                   ctypes.c_int, P, ctypes.c_size_t, P]
    lib.batteries_tensor_product_backward_l3_noalloc.restype = ctypes.c_int
    lib.batteries_tensor_product_backward_l3_noalloc.argtypes = [P] * 7 + [
        ctypes.c_int64, ctypes.c_int, ctypes.c_int, P]
    return lib


def _inputs(n, cin, cout, seed, dev):
    x = torch.randn(n, cin, 16, generator=gen(seed))
    y = torch.randn(n, 16, generator=gen(seed + 1))
    w = torch.randn(34, cin, cout, generator=gen(seed + 2)) / np.sqrt(cin)
    g = torch.randn(n, cout, 16, generator=gen(seed + 3))
    return [t.to(dev) for t in (x, y, w, g)]


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _run(lib, noalloc, x, y, w, g, dev):
    n, cin = x.shape[0], x.shape[1]
    cout = w.shape[2]
    gx = torch.full((n, cin, 16), float("nan"), device=dev)
    gy = torch.full((n, 16), float("nan"), device=dev)
    gw = torch.full((34, cin, cout), float("nan"), device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = [_ptr(x), _ptr(y), _ptr(w), _ptr(g), _ptr(gx), _ptr(gy), _ptr(gw), n, cin, cout]
    if noalloc:
        rc = lib.batteries_tensor_product_backward_l3_noalloc(*args, stream)
    else:
        wsb = lib.batteries_tensor_product_backward_workspace_bytes(n, cin, cout)
        ws = torch.empty((wsb + 3) // 4, device=dev)
        rc = lib.batteries_tensor_product_backward_l3(*args, _ptr(ws), wsb, stream)
    torch.cuda.synchronize()
    assert rc == 0
    return gx, gy, gw


def test_noalloc_backward_equals_workspace_backward(dev):
    lib = _lib()
    # configs[2]-like, then a smaller call: the scratch keeps the first call's partials,
    # which the second must not pick up
    for n, cin, cout, seed in [(6000, 32, 64, 501), (700, 16, 24, 511)]:
        print(f"noalloc backward n={n} cin={cin} cout={cout} seed={seed}", flush=True)
        assert lib.batteries_tensor_product_backward_workspace_bytes(n, cin, cout) <= SCRATCH_BYTES
        x, y, w, g = _inputs(n, cin, cout, seed, dev)
        ref = _run(lib, False, x, y, w, g, dev)
        got = _run(lib, True, x, y, w, g, dev)
        for a, b in zip(ref, got):
            assert torch.equal(a, b)
        # and the oracle on the first rows' grad_x / grad_y (rows are independent)
        k = 200
        wx, wy, _ = otp.tensor_product_backward(*(t[:k].cpu().double().numpy() if i != 2 else
                                                  t.cpu().double().numpy()
                                                  for i, t in enumerate((x, y, w, g))))
        assert normwise_err(got[0][:k].cpu(), wx) <= 1e-4
        assert normwise_err(got[1][:k].cpu(), wy) <= 1e-4


def test_noalloc_backward_weight_grad_against_oracle(dev):
    lib = _lib()
    n, cin, cout = 300, 8, 16
    x, y, w, g = _inputs(n, cin, cout, 521, dev)
    _, _, gw = _run(lib, True, x, y, w, g, dev)
    _, _, ww = otp.tensor_product_backward(*(t.cpu().double().numpy() for t in (x, y, w, g)))
    assert normwise_err(gw.cpu(), ww) <= 1e-4


def test_noalloc_backward_rejects_sizes_over_the_scratch(dev):
    lib = _lib()
    n, cin, cout = 100000, 1024, 1024   # 3 * 64 * 16 combos > 512: one segment of 142.6 MB
    assert lib.batteries_tensor_product_backward_workspace_bytes(n, cin, cout) > SCRATCH_BYTES
    dummy = torch.empty(16, device=dev)
    p = _ptr(dummy)
    rc = lib.batteries_tensor_product_backward_l3_noalloc(p, p, p, p, None, None, p, n, cin, cout,
                                                          None)
    assert rc == ERR_SCRATCH
    # without grad_weights no scratch is needed; empty N returns at once
    rc = lib.batteries_tensor_product_backward_l3_noalloc(p, p, p, p, None, None, None, 0, cin,
                                                          cout, None)
    assert rc == 0
