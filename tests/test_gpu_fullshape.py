"""GPU parity of the decode GEMVs at the exact 7B and 0.5B matrix shapes.

Same test as the reference's differential GEMV check
(crates/whetstone-kernels/tests/decode_kernels.rs:491-557: the kernel against
a float64 product of the dequantised matrix), at the configurations' own
shapes instead of row slices:

  7B  qkv 3584 -> 4608, gate|up 3584 -> 2*18944 (and its SwiGLU form),
      down 18944 -> 3584, lm_head 3584 -> 152064 (the two-units-in-flight head
      path, and its RMSNorm-prologue form)
  0.5B fp16 head 896 -> 151936 (wst_gemv_fp16) and the fp16 embedding row.

Weights are N(0, 0.02) packed on the device by the fixture packer (byte-equal
to the oracle's quantiser, tests/test_gpu_fixture_fused.py), copied back, and
dequantised on the host by the oracle (bit-exact with hier.rs:398-421).
"""
import numpy as np
import pytest

from conftest import dev_f16, f16
from whetstone_amd import ffi

pytestmark = pytest.mark.gpu


def _packed(orc, wk, in_f, out_f, stream):
    qw = wk.DeviceBuffer(out_f * in_f // 8, np.uint32)
    si = wk.DeviceBuffer(out_f * in_f // 32, np.uint8)
    sb = wk.DeviceBuffer(out_f, np.uint32)
    ffi.call("wst_fixture_pack_hier", qw.ptr, si.ptr, sb.ptr, in_f, 0, out_f, 0, stream, 0.02)
    host = orc.Packed(qw.numpy(), si.numpy(), sb.numpy(), in_f, out_f)
    return (qw, si, sb), host


def _reference(orc, p, xb, rows=8192):
    """float64 dequant(W) @ x, the scale sum |w||x|, and the same product with
    x rounded to the kernel's 14-bit activation table (oracle xq14)."""
    x = orc.f16_value(xb).astype(np.float64)
    xq = orc.xq14(xb)
    y, s, yq = (np.empty(p.out_f) for _ in range(3))
    w8, g = p.in_f // 8, p.in_f // 32
    for r0 in range(0, p.out_f, rows):
        r1 = min(p.out_f, r0 + rows)
        part = orc.Packed(p.qw[r0 * w8:r1 * w8], p.si[r0 * g:r1 * g], p.sb[r0:r1], p.in_f, r1 - r0)
        w = orc.dequantize(part).astype(np.float64)
        y[r0:r1] = w @ x
        yq[r0:r1] = w @ xq
        s[r0:r1] = np.abs(w) @ np.abs(x)
    return y, s, yq


def _x(orc, n, seed):
    return f16(orc, np.random.default_rng(seed).standard_normal(n).astype(np.float32))


@pytest.mark.parametrize("in_f,out_f", [(3584, 4608), (3584, 37888), (18944, 3584),
                                        (3584, 152064)],
                         ids=["7b-qkv", "7b-gate_up", "7b-down", "7b-lm_head"])
def test_gemv_full_shape_matches_float64(orc, wk, in_f, out_f):
    (qw, si, sb), p = _packed(orc, wk, in_f, out_f, 40 + in_f % 7 + out_f % 5)
    xb = _x(orc, in_f, out_f)
    xd = dev_f16(wk, xb)
    yd = wk.DeviceBuffer(out_f, np.float32)
    ffi.call("wst_gemv_int4_hier_ex", qw.ptr, si.ptr, sb.ptr, xd.ptr, None, yd.ptr, in_f, out_f, 0)
    got = yd.numpy().astype(np.float64)
    want, scale, want_q = _reference(orc, p, xb)
    err = np.abs(got - want) / np.maximum(scale, 1.0)
    print(f"{in_f}x{out_f}: worst {err.max():.3g} of sum|wx|")
    assert err.max() < 1e-4, f"worst {err.max():.3g} at row {err.argmax()}"
    # Against the product with the activation table's rounding, only f32
    # rounding of the per-group combination remains.
    errq = np.abs(got - want_q) / np.maximum(scale, 1.0)
    assert errq.max() < 2e-5, f"vs xq14: worst {errq.max():.3g} at row {errq.argmax()}"


def test_swiglu_form_full_7b_shape(orc, wk):
    in_f, inter = 3584, 18944
    (qw, si, sb), p = _packed(orc, wk, in_f, 2 * inter, 51)
    xb = _x(orc, in_f, 52)
    xd = dev_f16(wk, xb)
    act = wk.DeviceBuffer(inter, np.float16)
    ffi.call("wst_gemv_hier_swiglu", qw.ptr, si.ptr, sb.ptr, xd.ptr, None, 1e-6, act.ptr, in_f,
             inter)
    # bit-identical to the unfused ABI pair
    gu = wk.DeviceBuffer(2 * inter, np.float32)
    ffi.call("wst_gemv_int4_hier_ex", qw.ptr, si.ptr, sb.ptr, xd.ptr, None, gu.ptr, in_f,
             2 * inter, 0)
    act2 = wk.DeviceBuffer(inter, np.float16)
    ffi.call("wst_swiglu", gu.ptr, act2.ptr, inter)
    got = act.numpy()
    assert np.array_equal(got.view(np.uint16), act2.numpy().view(np.uint16))
    # and within f16 rounding (plus the GEMV bound) of the float64 form
    y, s, _ = _reference(orc, p, xb)
    g, u = y[:inter], y[inter:]
    want = g / (1 + np.exp(-g)) * u
    tol = 2.0 ** -10 * np.abs(want) + 1e-4 * (s[:inter] * np.abs(u) + s[inter:] * np.abs(g)) + 1e-6
    assert np.all(np.abs(got.astype(np.float64) - want) <= tol)


def test_rmsnorm_head_form_full_7b_shape(orc, wk):
    """The engine's head: final RMSNorm fused into the 3584 -> 152064 GEMV,
    bit-identical to wst_rmsnorm + wst_gemv_int4_hier_ex, argmax bit-exact."""
    in_f, vocab = 3584, 152064
    (qw, si, sb), p = _packed(orc, wk, in_f, vocab, 61)
    rng = np.random.default_rng(62)
    x = (rng.standard_normal(in_f) * 3).astype(np.float32)
    nw = f16(orc, 1 + 0.02 * rng.standard_normal(in_f))
    xd, nwd = wk.DeviceBuffer.from_array(x), dev_f16(wk, nw)
    y1, h1 = wk.DeviceBuffer(vocab, np.float32), wk.DeviceBuffer(in_f, np.float16)
    ffi.call("wst_gemv_hier_rmsnorm", qw.ptr, si.ptr, sb.ptr, xd.ptr, nwd.ptr, 1e-6, h1.ptr, None,
             y1.ptr, in_f, vocab, 0)
    h2, y2 = wk.DeviceBuffer(in_f, np.float16), wk.DeviceBuffer(vocab, np.float32)
    ffi.call("wst_rmsnorm", xd.ptr, nwd.ptr, h2.ptr, in_f, 1e-6)
    ffi.call("wst_gemv_int4_hier_ex", qw.ptr, si.ptr, sb.ptr, h2.ptr, None, y2.ptr, in_f, vocab, 0)
    assert np.array_equal(h1.numpy().view(np.uint16), h2.numpy().view(np.uint16))
    assert np.array_equal(y1.numpy().view(np.uint32), y2.numpy().view(np.uint32))
    assert np.array_equal(h1.numpy().view(np.uint16), orc.rmsnorm(x, nw, 1e-6))
    got = y1.numpy()
    want, scale, _ = _reference(orc, p, h1.numpy().view(np.uint16))
    assert np.max(np.abs(got - want) / np.maximum(scale, 1.0)) < 1e-4
    idx = wk.DeviceBuffer(1, np.int32)
    ffi.call("wst_argmax", y1.ptr, idx.ptr, vocab)
    assert int(idx.numpy()[0]) == orc.argmax(got)


def test_fp16_head_gemv_full_05b_shape(orc, wk):
    """wst_gemv_fp16 on the 0.5B tied head, 896 -> 151936: f16 weights and x
    are exact inputs, so only the f32 accumulation differs from float64."""
    in_f, out_f = 896, 151936
    w = wk.DeviceBuffer(out_f * in_f, np.float16)
    ffi.call("wst_fixture_normal_f16", w.ptr, out_f * in_f, 0, 71, 0, 0.02, 0.0)
    xb = _x(orc, in_f, 72)
    xd = dev_f16(wk, xb)
    y = wk.DeviceBuffer(out_f, np.float32)
    ffi.call("wst_gemv_fp16", w.ptr, xd.ptr, y.ptr, in_f, out_f)
    wf = w.numpy().astype(np.float64).reshape(out_f, in_f)
    xf = orc.f16_value(xb).astype(np.float64)
    want = wf @ xf
    bound = 1e-5 * (np.abs(wf) @ np.abs(xf)) + 1e-7
    got = y.numpy().astype(np.float64)
    assert np.all(np.abs(got - want) <= bound), float(np.max(np.abs(got - want) / bound))
    # the f16 embedding row is the table row widened, bit for bit, row clamped
    out = wk.DeviceBuffer(in_f, np.float32)
    table = w.numpy().reshape(out_f, in_f)
    for tok, row in [(0, 0), (123456, 123456), (out_f - 1, out_f - 1), (-3, 0), (10 ** 7, out_f - 1)]:
        cur = wk.DeviceCursor(tok)
        ffi.call("wst_embed_fp16", w.ptr, cur.buf.ptr, out.ptr, in_f, out_f)
        assert np.array_equal(out.numpy(), table[row].astype(np.float32)), tok


@pytest.mark.parametrize("k", [32, 64])
def test_head_rescore_full_05b_shape_against_oracle(orc, wk, k):
    """The config-4 head: the int4 logits of the 0.5B tied head (896 -> 151936)
    from the device GEMV, then the fused rescore from the fp16 copy (top k)
    against the oracle's ladder (orc_head_threshold, head_rescore.cu:62-180)
    and its f64 rescore of every row at or above the threshold
    (orc_head_rescore): the same threshold and count, rows below it
    untouched, rescored rows within f32 rounding of the f64 dot product."""
    in_f, vocab = 896, 151936
    w32 = wk.DeviceBuffer(vocab * in_f, np.float32)
    ffi.call("wst_fixture_normal_f32", w32.ptr, vocab * in_f, 0, 91, 0, 0.02)
    head16 = wk.DeviceBuffer(vocab * in_f, np.float16)  # the fp16 copy of the same weights
    ffi.call("wst_fixture_normal_f16", head16.ptr, vocab * in_f, 0, 91, 0, 0.02, 0.0)
    qw = wk.DeviceBuffer(vocab * in_f // 8, np.uint32)
    si = wk.DeviceBuffer(vocab * in_f // 32, np.uint8)
    sb = wk.DeviceBuffer(vocab, np.uint32)
    ffi.call("wst_quantize_int4_hier", w32.ptr, qw.ptr, si.ptr, sb.ptr, in_f, vocab)
    del w32
    xb = _x(orc, in_f, 92)
    xd = dev_f16(wk, xb)
    lg = wk.DeviceBuffer(vocab, np.float32)
    ffi.call("wst_gemv_int4_hier_ex", qw.ptr, si.ptr, sb.ptr, xd.ptr, None, lg.ptr, in_f, vocab, 0)
    approx = lg.numpy().copy()
    rs = wk.HeadRescore(head16, vocab, in_f, k)
    ffi.call("wst_head_rescore_fused", head16.ptr, xd.ptr, lg.ptr, vocab, in_f, k, rs.cap,
             rs.scratch.ptr, rs.nblocks)
    got = lg.numpy()
    th, cnt, _ = orc.head_threshold(approx, k, rs.cap)
    assert k <= cnt <= rs.cap
    want = approx.copy()
    hb = head16.numpy().view(np.uint16)
    orc.lib().orc_head_rescore(np.ascontiguousarray(hb), np.ascontiguousarray(xb), want, vocab,
                               in_f, np.float32(th))
    sel = approx >= th
    assert int(sel.sum()) == cnt
    np.testing.assert_array_equal(got[~sel], approx[~sel])
    rows = np.nonzero(sel)[0]
    h = orc.f16_value(hb.reshape(vocab, in_f)[rows].ravel()).astype(np.float64).reshape(-1, in_f)
    scale = np.abs(h) @ np.abs(orc.f16_value(xb).astype(np.float64))
    assert np.all(np.abs(got[sel].astype(np.float64) - want[sel]) <= 1e-5 * scale + 1e-6)
    assert int(np.argmax(got)) == int(np.argmax(want))
