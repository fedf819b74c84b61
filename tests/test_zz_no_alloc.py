"""wst_gemm_int4_hier_noalloc (the split-K chunk GEMM with its partials in a
static device array) against wst_gemm_int4_hier, through the C ABI.

Two calls in a row on the same GPU, the second with a smaller input, each
compared bit for bit with the allocating entry point on the same inputs (the
same kernels and the same split plan, so the same f32 sums in the same
order), and with a float64 product of the dequantised weights. Both shapes
split K (too few output tiles to fill the chip), so the static array is used.
"""
import numpy as np
import pytest

from conftest import dev_f16, f16
from whetstone_amd import ffi

pytestmark = pytest.mark.gpu


def _case(orc, wk, in_f, out_f, n, seed, accum):
    p, _ = orc.quantize(orc.fixture_normal(seed, 1, in_f * out_f), in_f, out_f)
    lin = wk.QuantLinearHier.from_packed(p)
    xb = f16(orc, orc.fixture_normal(seed, 2, n * in_f, 1.0))
    bias = f16(orc, orc.fixture_normal(seed, 3, out_f, 0.3))
    y0 = orc.fixture_normal(seed, 4, n * out_f, 1.0)
    xd, bd = dev_f16(wk, xb), dev_f16(wk, bias)
    ya = wk.DeviceBuffer.from_array(y0.copy())
    yb = wk.DeviceBuffer.from_array(y0.copy())
    ffi.call("wst_gemm_int4_hier", lin.qw.ptr, lin.si.ptr, lin.sb.ptr, xd.ptr, bd.ptr, ya.ptr,
             in_f, out_f, n, int(accum))
    ffi.call("wst_gemm_int4_hier_noalloc", lin.qw.ptr, lin.si.ptr, lin.sb.ptr, xd.ptr, bd.ptr,
             yb.ptr, in_f, out_f, n, int(accum))
    got, want = yb.numpy(), ya.numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    wd = orc.dequantize(p).astype(np.float64)
    xf = xb.view(np.float16).astype(np.float64).reshape(n, in_f)
    ref = xf @ wd.T + bias.view(np.float16).astype(np.float64)
    if accum:
        ref += y0.reshape(n, out_f)
    bound = 2.0 * 2.0 ** -11 * (np.abs(xf) @ np.abs(wd).T) + 1e-5 * (1 + np.abs(ref))
    assert np.all(np.abs(got.reshape(n, out_f) - ref) <= bound)


def test_noalloc_gemm_equals_allocating_gemm_twice(orc, wk):
    # the 0.5B down projection over a 256-token chunk: long rows, so the
    # 64 x 256 tiles, 14 of them, K split 16 ways (14.7 MB of partials)
    _case(orc, wk, 4864, 896, 256, 11, accum=True)
    # then a smaller input on the same static array: 64 x 64 tiles, K split
    _case(orc, wk, 896, 200, 37, 12, accum=False)


def test_noalloc_gemm_argument_checks(wk):
    st = ffi.lib().wst_gemm_int4_hier_noalloc(None, None, None, None, None, None, 32, 1, 1, 0)
    assert st == ffi.WST_ERR_INVALID_ARG
