"""GPU parity of jq_quantized_matmul_noalloc (the entry point whose K-split scratch is a fixed
device array of the library) against jq_quantized_matmul_ws with a caller workspace: bit
equality on two calls in a row, the second with a smaller input, and the size limit."""
import numpy as np
import pytest
import torch

from jangq_amd import _lib
from oracle import jangq_oracle as O
from tests._util import QWeight, assert_close, to_tensor, values_of

pytestmark = pytest.mark.gpu

LIMIT = 16 * 1024 * 1024  # JQ_NOALLOC_SCRATCH_BYTES


def _call_ws(lib, tx, qw, M, N, K, bits, gs):
    y = torch.empty((M, N), dtype=tx.dtype, device="cuda")
    nws = lib.jq_quantized_matmul_workspace_size(M, N, K, bits, gs, 1, 1)
    ws = torch.empty(max(nws, 256), dtype=torch.uint8, device="cuda")
    st = lib.jq_quantized_matmul_ws(tx.data_ptr(), 1, qw.dw.data_ptr(), qw.ds.data_ptr(),
                                    qw.db.data_ptr(), 1, bits, gs, M, N, K, y.data_ptr(), 1,
                                    ws.data_ptr(), ws.numel(),
                                    torch.cuda.current_stream().cuda_stream)
    assert st == 0
    return y, nws


def _call_static(lib, tx, qw, M, N, K, bits, gs):
    y = torch.empty((M, N), dtype=tx.dtype, device="cuda")
    st = lib.jq_quantized_matmul_noalloc(tx.data_ptr(), 1, qw.dw.data_ptr(), qw.ds.data_ptr(),
                                         qw.db.data_ptr(), 1, bits, gs, M, N, K, y.data_ptr(), 1,
                                         torch.cuda.current_stream().cuda_stream)
    return st, y


def test_noalloc_matches_workspace_form_twice():
    lib = _lib.lib()
    N, K, bits, gs = 4096, 14336, 2, 64   # config-2 down projection: the K-split shape
    qw = QWeight(N, K, bits, gs, seed=77)
    rng = np.random.default_rng(78)
    for M in (32, 9):  # the second call smaller: stale partials of the first must not leak
        x = O.round_bf16(rng.standard_normal((M, K), dtype=np.float32))
        tx = to_tensor(x, "bf16")
        ref, nws = _call_ws(lib, tx, qw, M, N, K, bits, gs)
        assert 0 < nws <= LIMIT
        st, y = _call_static(lib, tx, qw, M, N, K, bits, gs)
        assert st == 0
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), f"M={M}"
        exact = O.quantized_matmul(x[:4], qw.packed, qw.s, qw.b, bits, gs)
        assert_close(values_of(y)[:4], O.round_bf16(exact), f"noalloc M{M}", exact=exact,
                     out_dtype="bf16")


def test_noalloc_other_shapes_and_limit():
    lib = _lib.lib()
    # a shape without a split (decode GEMV): runs as jq_quantized_matmul
    qw = QWeight(256, 1024, 4, 64, seed=79)
    x = to_tensor(O.round_bf16(np.random.default_rng(80).standard_normal((1, 1024),
                                                                          dtype=np.float32)), "bf16")
    st, y = _call_static(lib, x, qw, 1, 256, 1024, 4, 64)
    ref, nws = _call_ws(lib, x, qw, 1, 256, 1024, 4, 64)
    assert st == 0 and nws == 0 and torch.equal(y, ref)
    # a split whose partials exceed the array: rejected before any launch
    M, N, K = 64, 65536, 8192
    need = lib.jq_quantized_matmul_workspace_size(M, N, K, 2, 64, 1, 1)
    assert need > LIMIT
    # full-size operands, so that the call would be in bounds even if it launched
    wc = torch.zeros((N, K * 2 // 32), dtype=torch.int32, device="cuda")
    sc = torch.zeros((N, K // 64), dtype=torch.bfloat16, device="cuda")
    xb = torch.zeros((M, K), dtype=torch.bfloat16, device="cuda")
    yb = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    st = lib.jq_quantized_matmul_noalloc(xb.data_ptr(), 1, wc.data_ptr(), sc.data_ptr(),
                                         sc.data_ptr(), 1, 2, 64, M, N, K, yb.data_ptr(), 1,
                                         torch.cuda.current_stream().cuda_stream)
    assert st == -7


def test_noalloc_prefill_runs_in_passes():
    """A prefill shape whose f16 activation rows exceed the array: the entry point runs them in
    passes of whole 256-row tiles, bit-equal to the workspace form with a full workspace, on
    two calls in a row (the second smaller)."""
    lib = _lib.lib()
    N, K, bits, gs = 1024, 4096, 4, 64
    qw = QWeight(N, K, bits, gs, seed=81)
    rng = np.random.default_rng(82)
    for M in (2304, 1100):
        x = O.round_bf16(rng.standard_normal((M, K), dtype=np.float32))
        tx = to_tensor(x, "bf16")
        ref, nws = _call_ws(lib, tx, qw, M, N, K, bits, gs)
        if M == 2304:
            assert nws > LIMIT  # the array holds fewer rows than the call has
        st, y = _call_static(lib, tx, qw, M, N, K, bits, gs)
        assert st == 0
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), f"M={M}"
        exact = O.quantized_matmul(x[-3:], qw.packed, qw.s, qw.b, bits, gs)
        assert_close(values_of(y)[-3:], O.round_bf16(exact), f"noalloc prefill M{M}",
                     exact=exact, out_dtype="bf16")
