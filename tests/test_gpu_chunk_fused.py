"""The fused chunk (prefill) forms against the unfused ABI sequence they
replace, bit for bit: gate|up GEMM + SwiGLU, GEMM + split reduce + RMSNorm,
qkv GEMM + split reduce + QK-norm/RoPE/KV append. Each fused form computes
the same expressions in the same order as the kernels it replaces (the GEMM
tile is unchanged; only where its result goes differs), so any difference is
a bug, not rounding. The unfused sequence itself is checked against float64
in test_gpu_kernels.py."""
import numpy as np
import pytest

from conftest import dev_f16, f16
from whetstone_amd import ffi

pytestmark = pytest.mark.gpu


def _lin(orc, wk, seed, in_f, out_f):
    p, _ = orc.quantize(orc.fixture_normal(seed, 1, in_f * out_f), in_f, out_f)
    return wk.QuantLinearHier.from_packed(p)


def _x(orc, wk, seed, n, in_f, std=1.0):
    return dev_f16(wk, f16(orc, orc.fixture_normal(seed, 2, n * in_f, std)))


@pytest.mark.parametrize("in_f,inter,n,exact,step", [(896, 4864, 256, True, 256),
                                                     (64, 33, 1, True, 256),
                                                     (128, 4096, 300, True, 256),
                                                     (3584, 100, 37, False, 256),
                                                     (896, 16640, 512, True, 512)])
def test_gemm_swiglu_chunk_equals_gemm_then_swiglu(orc, wk, in_f, inter, n, exact, step):
    """Bit for bit where the unfused GEMM runs unsplit (an output tile's sum in
    one K order). The fused form never splits K; where the unfused one does
    (few output tiles: the fourth case), its f32 sums are added in another
    order, and the f16 outputs may differ in the last place. The last case
    runs 512 tokens in one call, as a batched prefill does: 260 x 2 tiles of
    128 rows, so both forms take the 128-row wide tiles."""
    lin = _lin(orc, wk, 21, in_f, 2 * inter)
    x = _x(orc, wk, 22, n, in_f)
    gu = wk.DeviceBuffer(n * 2 * inter, np.float32)
    want = wk.DeviceBuffer(n * inter, np.float16)
    got = wk.DeviceBuffer(n * inter, np.float16)
    for j in range(0, n, step):  # chunks of at most `step` tokens
        m = min(step, n - j)
        xo = x.ptr.value + j * in_f * 2
        ffi.call("wst_gemm_int4_hier", lin.qw.ptr, lin.si.ptr, lin.sb.ptr, xo, None, gu.ptr,
                 in_f, 2 * inter, m, 0)
        ffi.call("wst_swiglu_chunk", gu.ptr, want.ptr.value + j * inter * 2, inter, m)
        ffi.call("wst_gemm_hier_swiglu_chunk", lin.qw.ptr, lin.si.ptr, lin.sb.ptr, xo,
                 got.ptr.value + j * inter * 2, in_f, inter, m)
    a, b = want.numpy().view(np.uint16), got.numpy().view(np.uint16)
    if exact:
        assert np.array_equal(a, b), int(np.sum(a != b))
    else:
        fa, fb = a.view(np.float16).astype(np.float64), b.view(np.float16).astype(np.float64)
        assert np.all(np.abs(fa - fb) <= 2.0 ** -10 * np.abs(fa) + 1e-3), float(np.max(np.abs(fa - fb)))


@pytest.mark.parametrize("in_f,out_f,n,accum,bias", [(896, 896, 256, 1, False),
                                                     (4864, 896, 256, 1, False),
                                                     (3584, 3584, 37, 0, True),
                                                     (96, 70, 5, 1, True),
                                                     (1536, 1536, 9, 1, True),
                                                     (256, 4100, 3, 0, False)])
def test_gemm_norm_chunk_equals_gemm_then_rmsnorm(orc, wk, in_f, out_f, n, accum, bias):
    lin = _lin(orc, wk, 31, in_f, out_f)
    x = _x(orc, wk, 32, n, in_f)
    b = dev_f16(wk, f16(orc, orc.fixture_normal(31, 3, out_f, 0.3))) if bias else None
    nw = dev_f16(wk, f16(orc, 1.0 + orc.fixture_normal(31, 4, out_f, 0.1)))
    y0 = orc.fixture_normal(31, 5, n * out_f, 1.0)
    ya, yb = wk.DeviceBuffer.from_array(y0.copy()), wk.DeviceBuffer.from_array(y0.copy())
    ha, hb = wk.DeviceBuffer(n * out_f, np.float16), wk.DeviceBuffer(n * out_f, np.float16)
    bp = b.ptr if b is not None else None
    ffi.call("wst_gemm_int4_hier", lin.qw.ptr, lin.si.ptr, lin.sb.ptr, x.ptr, bp, ya.ptr, in_f,
             out_f, n, accum)
    ffi.call("wst_rmsnorm_chunk", ya.ptr, nw.ptr, ha.ptr, out_f, n, 1e-6)
    ffi.call("wst_gemm_hier_norm_chunk", lin.qw.ptr, lin.si.ptr, lin.sb.ptr, x.ptr, bp, yb.ptr,
             in_f, out_f, n, accum, nw.ptr, 1e-6, hb.ptr)
    assert np.array_equal(ya.numpy().view(np.uint32), yb.numpy().view(np.uint32))
    assert np.array_equal(ha.numpy().view(np.uint16), hb.numpy().view(np.uint16))


@pytest.mark.parametrize("in_f,n_q,n_kv,hd,pos0,n,qk,has_bias",
                         [(896, 14, 2, 64, 0, 256, False, True),
                          (896, 14, 2, 64, 300, 256, True, True),
                          (3584, 28, 4, 128, 5, 37, False, True),
                          (512, 8, 2, 128, 60, 3, True, True),
                          (896, 14, 2, 64, 0, 2048, True, True),
                          (896, 14, 2, 64, 100, 2000, False, True),
                          (896, 14, 2, 64, 6, 2050, True, False)])
def test_gemm_rope_chunk_equals_gemm_then_rope_cache(orc, wk, in_f, n_q, n_kv, hd, pos0, n, qk,
                                                     has_bias):
    """The fused qkv form against the GEMM then wst_rope_cache_chunk, bit for
    bit (q rotated, k and v as computed, the cache rows). At head_dim 64 with
    about 1800 tokens or more the GEMM runs unsplit on 256-token tiles, one
    head a tile, and the tile's epilogue does the norm, rotation and append
    (the last three cases: one with a ragged last tile, one without a bias,
    as Qwen3's projections have none, ending at the cache's last row); below
    that a reduce kernel does them after the GEMM."""
    out_f = (n_q + 2 * n_kv) * hd
    max_seq = pos0 + n + (7 if has_bias else 0)
    lin = _lin(orc, wk, 41, in_f, out_f)
    x = _x(orc, wk, 42, n, in_f)
    b = dev_f16(wk, f16(orc, orc.fixture_normal(41, 3, out_f, 0.3))) if has_bias else None
    bp = b.ptr if has_bias else None
    qn = dev_f16(wk, f16(orc, 1.0 + orc.fixture_normal(41, 4, hd, 0.1))) if qk else None
    kn = dev_f16(wk, f16(orc, 1.0 + orc.fixture_normal(41, 5, hd, 0.1))) if qk else None
    c, s = orc.rope_table(max_seq, hd, 1e6)
    cd, sd = wk.DeviceBuffer.from_array(c), wk.DeviceBuffer.from_array(s)
    kv0 = f16(orc, orc.fixture_normal(41, 6, n_kv * max_seq * hd, 1.0))
    bufs = []
    for _ in range(2):
        bufs.append((wk.DeviceBuffer(n * out_f, np.float32), dev_f16(wk, kv0), dev_f16(wk, kv0)))
    qp, kp = (qn.ptr if qk else None), (kn.ptr if qk else None)
    (qa, ka, va), (qb, kb, vb) = bufs
    ffi.call("wst_gemm_int4_hier", lin.qw.ptr, lin.si.ptr, lin.sb.ptr, x.ptr, bp, qa.ptr, in_f,
             out_f, n, 0)
    ffi.call("wst_rope_cache_chunk", qa.ptr, ka.ptr, va.ptr, cd.ptr, sd.ptr, n_q, n_kv, hd, pos0,
             n, max_seq, qp, kp, 1e-6)
    ffi.call("wst_gemm_hier_rope_chunk", lin.qw.ptr, lin.si.ptr, lin.sb.ptr, x.ptr, bp,
             qb.ptr, in_f, kb.ptr, vb.ptr, cd.ptr, sd.ptr, n_q, n_kv, hd, pos0, n, max_seq, qp,
             kp, 1e-6)
    assert np.array_equal(qa.numpy().view(np.uint32), qb.numpy().view(np.uint32))
    assert np.array_equal(ka.numpy().view(np.uint16), kb.numpy().view(np.uint16))
    assert np.array_equal(va.numpy().view(np.uint16), vb.numpy().view(np.uint16))
    # the chunk's rows were written; the rest of the cache is untouched
    k = kb.numpy().view(np.uint16).reshape(n_kv, max_seq, hd)
    k0 = kv0.reshape(n_kv, max_seq, hd)
    assert np.array_equal(k[:, :pos0], k0[:, :pos0]) and np.array_equal(k[:, pos0 + n:], k0[:, pos0 + n:])


def test_fused_chunk_forms_refuse_bad_shapes(orc, wk):
    lin = _lin(orc, wk, 51, 64, 64)
    x = _x(orc, wk, 52, 4, 64)
    y = wk.DeviceBuffer(4 * 64, np.float32)
    h = wk.DeviceBuffer(4 * 64, np.float16)
    with pytest.raises(ffi.WstError):  # null norm weight
        ffi.call("wst_gemm_hier_norm_chunk", lin.qw.ptr, lin.si.ptr, lin.sb.ptr, x.ptr, None,
                 y.ptr, 64, 64, 4, 0, None, 1e-6, h.ptr)
    with pytest.raises(ffi.WstError):  # in_f not a multiple of 32
        ffi.call("wst_gemm_hier_swiglu_chunk", lin.qw.ptr, lin.si.ptr, lin.sb.ptr, x.ptr, h.ptr,
                 48, 32, 4)
    with pytest.raises(ffi.WstError):  # head_dim above 128
        ffi.call("wst_gemm_hier_rope_chunk", lin.qw.ptr, lin.si.ptr, lin.sb.ptr, x.ptr, None,
                 y.ptr, 64, h.ptr, h.ptr, y.ptr, y.ptr, 1, 1, 256, 0, 1, 8, None, None, 1e-6)
