"""GPU tests of the device fixture generator / packer (bit-exact against the
host quantiser restatement of hier.rs) and of the fused decode-step kernels
(bit-exact against the unfused ABI sequence they replace)."""
import math

import numpy as np
import pytest

from conftest import dev_f16, f16
from whetstone_amd import ffi

pytestmark = pytest.mark.gpu


def test_fixture_normal_is_bit_exact(orc, wk):
    n = 100003
    d = wk.DeviceBuffer(n, np.float32)
    ffi.call("wst_fixture_normal_f32", d.ptr, n, 7, 123, 5000, np.float32(0.02))
    want = orc.fixture_normal(7, 123, n, 0.02, index0=5000)
    assert np.array_equal(d.numpy().view(np.uint32), want.view(np.uint32))
    h = wk.DeviceBuffer(n, np.float16)
    ffi.call("wst_fixture_normal_f16", h.ptr, n, 7, 124, 0, np.float32(0.02), np.float32(1.0))
    want = f16(orc, np.float32(1.0) + orc.fixture_normal(7, 124, n, 0.02))
    assert np.array_equal(h.numpy().view(np.uint16), want)


@pytest.mark.parametrize("in_f,rows", [(896, 257), (4864, 33), (3584, 40), (18944, 5), (64, 9)])
def test_device_packer_matches_host_quantiser(orc, wk, in_f, rows):
    qw = wk.DeviceBuffer(rows * in_f // 8, np.uint32)
    si = wk.DeviceBuffer(rows * in_f // 32, np.uint8)
    sb = wk.DeviceBuffer(rows, np.uint32)
    ffi.call("wst_fixture_pack_hier", qw.ptr, si.ptr, sb.ptr, in_f, 0, rows, 11, 77,
             np.float32(0.02))
    w = orc.fixture_normal(11, 77, rows * in_f, 0.02)
    p, _ = orc.quantize(w, in_f, rows)
    assert np.array_equal(sb.numpy(), p.sb)
    assert np.array_equal(si.numpy(), p.si)
    assert np.array_equal(qw.numpy(), p.qw)


def test_device_packer_on_adversarial_rows(orc, wk):
    """The quantiser's edge cases (hier.rs:467-557): a group with a huge range
    next to near-constant groups, constant and zero rows, rows so small that
    the shared f16 scale would underflow, large magnitudes."""
    in_f = 256
    rows = []
    r = np.full(in_f, 1e-6, np.float32)
    r[:32] = -40.0
    r[0] = 40.0
    rows.append(r)
    rows.append(np.zeros(in_f, np.float32))
    rows.append(np.full(in_f, 0.25, np.float32))
    rows.append(np.full(in_f, -0.5, np.float32))
    rows.append((((np.arange(in_f) % 17) - 8.0) * 1e-10).astype(np.float32))
    rows.append((((np.arange(in_f) % 17) - 8.0) * 0.01).astype(np.float32))
    rows.append((np.sin(np.arange(in_f)) * 3e4).astype(np.float32))
    rng = np.random.default_rng(1)
    rows.append((rng.standard_normal(in_f) ** 3).astype(np.float32))
    w = np.stack(rows)
    n = w.shape[0]
    wd = wk.DeviceBuffer.from_array(w.ravel())
    qw = wk.DeviceBuffer(n * in_f // 8, np.uint32)
    si = wk.DeviceBuffer(n * in_f // 32, np.uint8)
    sb = wk.DeviceBuffer(n, np.uint32)
    ffi.call("wst_quantize_int4_hier", wd.ptr, qw.ptr, si.ptr, sb.ptr, in_f, n)
    p, _ = orc.quantize(w.ravel(), in_f, n)
    assert np.array_equal(sb.numpy(), p.sb)
    assert np.array_equal(si.numpy(), p.si)
    assert np.array_equal(qw.numpy(), p.qw)


def test_fill_kv_matches_oracle(orc, wk):
    n_kv, max_seq, hd, n = 2, 40, 64, 33
    k = wk.DeviceBuffer(n_kv * max_seq * hd, np.float16)
    v = wk.DeviceBuffer(n_kv * max_seq * hd, np.float16)
    ffi.call("wst_fixture_fill_kv", k.ptr, v.ptr, n_kv, max_seq, hd, n, 5, 1003)
    kk = k.numpy().view(np.uint16).reshape(n_kv, max_seq, hd)
    vv = v.numpy().view(np.uint16).reshape(n_kv, max_seq, hd)
    for h in range(n_kv):
        for kv, arr in ((0, kk), (1, vv)):
            for t in (0, 17, n - 1):
                base = (((h * 2 + kv) << 20) + t) * hd
                want = f16(orc, orc.fixture_normal(5, 1003, hd, 1.0, index0=base))
                assert np.array_equal(arr[h, t], want)
    assert not kk[:, n:].any()


# ------------------------------------------------------------- fused kernels


@pytest.mark.parametrize("in_f,out_f", [(896, 1152), (3584, 520), (4864, 896)])
def test_gemv_rmsnorm_equals_rmsnorm_then_gemv(orc, wk, in_f, out_f):
    p, _ = orc.quantize(orc.fixture_normal(2, 1, in_f * out_f), in_f, out_f)
    lin = wk.QuantLinearHier.from_packed(p)
    x = orc.fixture_normal(2, 2, in_f, 3.0)
    nw = dev_f16(wk, f16(orc, 1.0 + orc.fixture_normal(2, 3, in_f, 0.1)))
    bias = dev_f16(wk, f16(orc, orc.fixture_normal(2, 4, out_f, 0.3)))
    xd = wk.DeviceBuffer.from_array(x)
    h = wk.DeviceBuffer(in_f, np.float16)
    y1 = wk.DeviceBuffer(out_f, np.float32)
    wk.rmsnorm(xd, nw, h, 1e-6)
    lin.gemv_ex(h, bias, y1)
    y2 = wk.DeviceBuffer(out_f, np.float32)
    h2 = wk.DeviceBuffer(in_f, np.float16)
    ffi.call("wst_gemv_hier_rmsnorm", lin.qw.ptr, lin.si.ptr, lin.sb.ptr, xd.ptr, nw.ptr,
             np.float32(1e-6), h2.ptr, bias.ptr, y2.ptr, in_f, out_f, 0)
    assert np.array_equal(y1.numpy().view(np.uint32), y2.numpy().view(np.uint32))
    assert np.array_equal(h.numpy().view(np.uint16), h2.numpy().view(np.uint16))


@pytest.mark.parametrize("in_f,inter,norm", [(896, 4864, True), (3584, 1000, True),
                                             (896, 300, False)])
def test_gemv_swiglu_equals_gemv_then_swiglu(orc, wk, in_f, inter, norm):
    p, _ = orc.quantize(orc.fixture_normal(3, 1, in_f * 2 * inter), in_f, 2 * inter)
    lin = wk.QuantLinearHier.from_packed(p)
    x = orc.fixture_normal(3, 2, in_f, 3.0)
    nw = dev_f16(wk, f16(orc, 1.0 + orc.fixture_normal(3, 3, in_f, 0.1)))
    xd = wk.DeviceBuffer.from_array(x)
    gu = wk.DeviceBuffer(2 * inter, np.float32)
    a1 = wk.DeviceBuffer(inter, np.float16)
    if norm:
        h = wk.DeviceBuffer(in_f, np.float16)
        wk.rmsnorm(xd, nw, h, 1e-6)
        src = xd
    else:
        h = dev_f16(wk, f16(orc, x))
        src = h
    lin.gemv(h, gu)
    wk.swiglu(gu, a1)
    a2 = wk.DeviceBuffer(inter, np.float16)
    ffi.call("wst_gemv_hier_swiglu", lin.qw.ptr, lin.si.ptr, lin.sb.ptr, src.ptr,
             nw.ptr if norm else None, np.float32(1e-6), a2.ptr, in_f, inter)
    assert np.array_equal(a1.numpy().view(np.uint16), a2.numpy().view(np.uint16))


@pytest.mark.parametrize("n_q,n_kv,hd,max_seq,pos,qkn", [(14, 2, 64, 1024, 600, False),
                                                         (28, 4, 128, 2304, 2100, False),
                                                         (14, 2, 64, 300, 0, True),
                                                         (16, 8, 128, 700, 511, True),
                                                         (28, 4, 128, 8192, 5000, True),
                                                         (14, 2, 64, 4168, 4100, True)])
def test_fused_attention_equals_rope_then_attention(orc, wk, n_q, n_kv, hd, max_seq, pos, qkn):
    rng = np.random.default_rng(pos + hd)
    qkv = (rng.standard_normal((n_q + 2 * n_kv) * hd) * 2).astype(np.float32)
    kc = f16(orc, rng.standard_normal(n_kv * max_seq * hd).astype(np.float32)).view(np.float16)
    vc = f16(orc, rng.standard_normal(n_kv * max_seq * hd).astype(np.float32)).view(np.float16)
    table = wk.RopeTable(max_seq, hd, 1e6)
    gq = dev_f16(wk, f16(orc, 1.0 + 0.1 * rng.standard_normal(hd)))
    gk = dev_f16(wk, f16(orc, 1.0 + 0.1 * rng.standard_normal(hd)))
    cur = wk.DeviceCursor(pos)
    # unfused
    c1 = wk.KvCache(n_kv, n_q, hd, max_seq)
    c1.k.copy_from(kc)
    c1.v.copy_from(vc)
    q1 = wk.DeviceBuffer.from_array(qkv)
    wk.rope_cache(q1, c1, table, n_q, cur, (gq, gk, 1e-6) if qkn else None)
    o1 = wk.DeviceBuffer(n_q * hd, np.float16)
    wk.attn_decode(q1, c1, o1, n_q, cur)
    # fused
    c2 = wk.KvCache(n_kv, n_q, hd, max_seq)
    c2.k.copy_from(kc)
    c2.v.copy_from(vc)
    q2 = wk.DeviceBuffer.from_array(qkv)
    o2 = wk.DeviceBuffer(n_q * hd, np.float16)
    ffi.call("wst_attn_decode_fused", q2.ptr, c2.k.ptr, c2.v.ptr, table.cos.ptr, table.sin.ptr,
             c2.partials.ptr, o2.ptr, n_q, n_kv, hd, cur.buf.ptr, max_seq,
             np.float32(1.0 / math.sqrt(hd)), gq.ptr if qkn else None,
             gk.ptr if qkn else None, np.float32(1e-6))
    assert np.array_equal(o1.numpy().view(np.uint16), o2.numpy().view(np.uint16))
    assert np.array_equal(c1.k.numpy().view(np.uint16), c2.k.numpy().view(np.uint16))
    assert np.array_equal(c1.v.numpy().view(np.uint16), c2.v.numpy().view(np.uint16))


def test_argmax_advance(orc, wk):
    v = np.random.default_rng(3).standard_normal(151936).astype(np.float32)
    idx = wk.DeviceBuffer(1, np.int32)
    pos = wk.DeviceCursor(10)
    vd = wk.DeviceBuffer.from_array(v)  # held: the launches are asynchronous
    ffi.call("wst_argmax_advance", vd.ptr, idx.ptr, v.size, pos.buf.ptr, 11)
    assert idx.numpy()[0] == orc.argmax(v) and pos.get() == 11
    ffi.call("wst_argmax_advance", vd.ptr, idx.ptr, v.size, pos.buf.ptr, 11)
    assert pos.get() == 11  # saturates at max_seq


def test_fused_rescore_equals_threshold_compact_rescore(orc, wk):
    vocab, hidden, k = 151936, 896, 64
    rng = np.random.default_rng(5)
    head = f16(orc, (rng.standard_normal(vocab * hidden) * 0.02).astype(np.float32))
    x = f16(orc, rng.standard_normal(hidden).astype(np.float32))
    logits = (rng.standard_normal(vocab) * 0.6).astype(np.float32)
    hd, xd = dev_f16(wk, head), dev_f16(wk, x)
    l1 = wk.DeviceBuffer.from_array(logits)
    rs = wk.HeadRescore(hd, vocab, hidden, k)
    rs.apply(l1, xd)
    l2 = wk.DeviceBuffer.from_array(logits)
    ffi.call("wst_head_rescore_fused", hd.ptr, xd.ptr, l2.ptr, vocab, hidden, k, rs.cap,
             rs.scratch.ptr, rs.nblocks)
    assert rs.last_count() <= rs.cap
    assert np.array_equal(l1.numpy().view(np.uint32), l2.numpy().view(np.uint32))


@pytest.mark.parametrize("n_q,n_kv,hd,max_seq,pos,out_f", [(14, 2, 64, 776, 700, 896),
                                                           (14, 2, 64, 776, 0, 896),
                                                           (8, 2, 128, 1024, 1023, 512),
                                                           (28, 4, 128, 600, 257, 3584),
                                                           (4, 2, 64, 2048, 1500, 96)])
def test_gemv_hier_attn_equals_merge_then_gemv(orc, wk, n_q, n_kv, hd, max_seq, pos, out_f):
    """wst_gemv_hier_attn (the slice merge inside the o GEMV) against
    wst_attn_decode (slices + merge kernel) followed by the plain GEMV, on the
    same partials: bit for bit, accumulating onto the same y."""
    from whetstone_amd import ffi
    rng = np.random.default_rng(pos + 3)
    kc = f16(orc, rng.standard_normal(n_kv * max_seq * hd).astype(np.float32))
    vc = f16(orc, rng.standard_normal(n_kv * max_seq * hd).astype(np.float32))
    q = wk.DeviceBuffer.from_array((rng.standard_normal(n_q * hd) * 2).astype(np.float32))
    cache = wk.KvCache(n_kv, n_q, hd, max_seq)
    cache.k.copy_from(kc.view(np.float16))
    cache.v.copy_from(vc.view(np.float16))
    cur = wk.DeviceCursor(pos)
    out = wk.DeviceBuffer(n_q * hd, np.float16)
    wk.attn_decode(q, cache, out, n_q, cur)
    in_f = n_q * hd
    p, _ = orc.quantize(orc.fixture_normal(9, 1, in_f * out_f), in_f, out_f)
    lin = wk.QuantLinearHier.from_packed(p)
    y0 = orc.fixture_normal(9, 2, out_f, 1.0)
    ya, yb = wk.DeviceBuffer.from_array(y0.copy()), wk.DeviceBuffer.from_array(y0.copy())
    ffi.call("wst_gemv_int4_hier_ex", lin.qw.ptr, lin.si.ptr, lin.sb.ptr, out.ptr, None, ya.ptr,
             in_f, out_f, 1)
    ffi.call("wst_gemv_hier_attn", lin.qw.ptr, lin.si.ptr, lin.sb.ptr, cache.partials.ptr,
             yb.ptr, n_q, hd, cur.buf.ptr, max_seq, out_f, 1)
    assert np.array_equal(ya.numpy().view(np.uint32), yb.numpy().view(np.uint32))


def test_gemv_hier_attn_refuses_long_caches(orc, wk):
    from whetstone_amd import ffi
    cache = wk.KvCache(2, 14, 64, 4096)  # 16 slices of 256 positions
    lin = wk.QuantLinearHier.from_packed(orc.quantize(orc.fixture_normal(9, 1, 896 * 64), 896, 64)[0])
    y = wk.DeviceBuffer(64, np.float32)
    with pytest.raises(ffi.WstError):
        ffi.call("wst_gemv_hier_attn", lin.qw.ptr, lin.si.ptr, lin.sb.ptr, cache.partials.ptr,
                 y.ptr, 14, 64, wk.DeviceCursor(5).buf.ptr, 4096, 64, 0)


@pytest.mark.parametrize("in_f,vocab", [(3584, 152064), (896, 151936), (256, 4096), (512, 40)])
def test_head_argmax_equals_head_then_argmax_advance(orc, wk, in_f, vocab):
    """wst_gemv_hier_rmsnorm_argmax against wst_gemv_hier_rmsnorm followed by
    wst_argmax_advance: the same logits bit for bit, the same token (planted
    ties between duplicated rows go to the lowest index), the same position."""
    qw = wk.DeviceBuffer(vocab * in_f // 8, np.uint32)
    si = wk.DeviceBuffer(vocab * in_f // 32, np.uint8)
    sb = wk.DeviceBuffer(vocab, np.uint32)
    ffi.call("wst_fixture_pack_hier", qw.ptr, si.ptr, sb.ptr, in_f, 0, vocab, 0, 81, 0.02)
    rng = np.random.default_rng(in_f + vocab)
    x = (rng.standard_normal(in_f) * 2).astype(np.float32)
    nw = f16(orc, 1 + 0.02 * rng.standard_normal(in_f))
    xd, nwd = wk.DeviceBuffer.from_array(x), dev_f16(wk, nw)
    # find the winning row, then copy it over a lower and a higher row: a tie
    y = wk.DeviceBuffer(vocab, np.float32)
    ffi.call("wst_gemv_hier_rmsnorm", qw.ptr, si.ptr, sb.ptr, xd.ptr, nwd.ptr, 1e-6, None, None,
             y.ptr, in_f, vocab, 0)
    top = int(np.argmax(y.numpy()))
    q, i_, b = qw.numpy(), si.numpy(), sb.numpy()
    for dst in {max(top - 7, 0), min(top + 5, vocab - 1)} - {top}:
        q[dst * in_f // 8:(dst + 1) * in_f // 8] = q[top * in_f // 8:(top + 1) * in_f // 8]
        i_[dst * in_f // 32:(dst + 1) * in_f // 32] = i_[top * in_f // 32:(top + 1) * in_f // 32]
        b[dst] = b[top]
    qw.copy_from(q), si.copy_from(i_), sb.copy_from(b)
    want_tok = min(max(top - 7, 0), top)
    y1, h1 = wk.DeviceBuffer(vocab, np.float32), wk.DeviceBuffer(in_f, np.float16)
    t1, p1 = wk.DeviceBuffer(1, np.int32), wk.DeviceCursor(100)
    ffi.call("wst_gemv_hier_rmsnorm", qw.ptr, si.ptr, sb.ptr, xd.ptr, nwd.ptr, 1e-6, h1.ptr, None,
             y1.ptr, in_f, vocab, 0)
    ffi.call("wst_argmax_advance", y1.ptr, t1.ptr, vocab, p1.buf.ptr, 102)
    for rep in range(3):  # repeated launches: the counter resets itself
        y2, h2 = wk.DeviceBuffer(vocab, np.float32), wk.DeviceBuffer(in_f, np.float16)
        t2, p2 = wk.DeviceBuffer(1, np.int32), wk.DeviceCursor(100 + rep)
        ffi.call("wst_gemv_hier_rmsnorm_argmax", qw.ptr, si.ptr, sb.ptr, xd.ptr, nwd.ptr, 1e-6,
                 h2.ptr, y2.ptr, in_f, vocab, t2.ptr, p2.buf.ptr, 102)
        assert np.array_equal(y1.numpy().view(np.uint32), y2.numpy().view(np.uint32))
        assert np.array_equal(h1.numpy().view(np.uint16), h2.numpy().view(np.uint16))
        assert int(t2.numpy()[0]) == int(t1.numpy()[0]) == want_tok == orc.argmax(y2.numpy())
        assert p2.get() == min(101 + rep, 102)
    assert p1.get() == 101
    t3 = wk.DeviceBuffer(1, np.int32)
    ffi.call("wst_gemv_hier_rmsnorm_argmax", qw.ptr, si.ptr, sb.ptr, xd.ptr, nwd.ptr, 1e-6,
             None, y2.ptr, in_f, vocab, t3.ptr, None, 0)   # no position to advance
    assert int(t3.numpy()[0]) == want_tok
