"""The int4-hier GEMV activation table built by a producer (the SwiGLU
gate|up GEMV, the attention merge, or wst_hier_xq_table) and consumed by
wst_gemv_hier_xq: every form gives the bits of the form that builds the table
inside the GEMV, and the table itself decodes to the oracle's 14-bit
activation values (orc_xq14)."""
import math

import numpy as np
import pytest

from conftest import dev_f16, f16
from whetstone_amd import ffi

pytestmark = pytest.mark.gpu

WORDS = 20  # u32 words per 32-column entry


def _decode(words, n):
    """Table words -> (value of each column, the entry's 8*sum, sum, scale)."""
    t = words.reshape(-1, WORDS)
    vals = np.empty(n, np.float64)
    for g in range(n // 32):
        e = t[g]
        sc = float(e[18:19].view(np.float32)[0])
        for k in range(4):
            for i in range(8):
                x = 0
                for j in range(4):
                    d = (int(e[4 * k + j]) >> (4 * i)) & 0xF
                    x += (d - 16 if d >= 8 else d) * 16 ** j
                vals[32 * g + 8 * k + i] = x * sc
    return vals, t[:, 16].view(np.int32), t[:, 17].view(np.float32), t[:, 18].view(np.float32)


def _table(wk, xd, n):
    t = wk.DeviceBuffer(n // 32 * WORDS, np.uint32)
    ffi.call("wst_hier_xq_table", xd.ptr, t.ptr, n)
    return t


def _same_entries(a, b):
    """Entries equal apart from the unused word 19."""
    a, b = a.reshape(-1, WORDS)[:, :19], b.reshape(-1, WORDS)[:, :19]
    return np.array_equal(a, b)


def test_table_decodes_to_the_oracle_xq14(orc, wk):
    rng = np.random.default_rng(4)
    n = 4096
    x = rng.standard_normal(n).astype(np.float32) * np.exp2(rng.integers(-20, 8, n)).astype(np.float32)
    x[:32] = 0.0                      # an all-zero group
    x[32:64] = 3e-7                   # f16 subnormals only
    x[64] = 65504.0                   # the f16 maximum beside small values
    x[96:128] = -1.0                  # a constant group
    xb = f16(orc, x)
    t = _table(wk, dev_f16(wk, xb), n).numpy()
    vals, c8, s, sc = _decode(t, n)
    want = orc.xq14(xb)
    assert np.array_equal(vals, want)
    xs = (want.reshape(-1, 32) / sc.astype(np.float64)[:, None]).sum(1)
    assert np.array_equal(c8, (8 * xs).astype(np.int32))
    assert np.array_equal(s.astype(np.float64), (xs * sc.astype(np.float64)).astype(np.float32))


@pytest.mark.parametrize("in_f,out_f,bias,accum", [(18944, 3584, False, 1), (3584, 3584, False, 1),
                                                   (4864, 896, False, 1), (896, 1152, True, 0),
                                                   (3584, 600, True, 1),
                                                   # head shapes: two units in flight, the
                                                   # second issued after the table's DMA
                                                   (896, 151936, False, 0),
                                                   (3584, 152064, False, 0)])
def test_gemv_on_a_table_equals_gemv_on_x(orc, wk, in_f, out_f, bias, accum):
    qw = wk.DeviceBuffer(out_f * in_f // 8, np.uint32)
    si = wk.DeviceBuffer(out_f * in_f // 32, np.uint8)
    sb = wk.DeviceBuffer(out_f, np.uint32)
    ffi.call("wst_fixture_pack_hier", qw.ptr, si.ptr, sb.ptr, in_f, 0, out_f, 0, 61, 0.02)
    rng = np.random.default_rng(in_f + out_f)
    xd = dev_f16(wk, f16(orc, rng.standard_normal(in_f).astype(np.float32)))
    bd = dev_f16(wk, f16(orc, rng.standard_normal(out_f).astype(np.float32))) if bias else None
    y0 = rng.standard_normal(out_f).astype(np.float32)
    y1, y2 = wk.DeviceBuffer.from_array(y0), wk.DeviceBuffer.from_array(y0)
    ffi.call("wst_gemv_int4_hier_ex", qw.ptr, si.ptr, sb.ptr, xd.ptr, bd.ptr if bias else None,
             y1.ptr, in_f, out_f, accum)
    t = _table(wk, xd, in_f)
    ffi.call("wst_gemv_hier_xq", qw.ptr, si.ptr, sb.ptr, t.ptr, bd.ptr if bias else None, y2.ptr,
             in_f, out_f, accum)
    assert np.array_equal(y1.numpy().view(np.uint32), y2.numpy().view(np.uint32))


@pytest.mark.parametrize("in_f,inter,norm", [(3584, 18944, True), (896, 4864, True),
                                             (3584, 1024, True), (896, 320, False),
                                             # rows of two waves (4 and 8 rows per block
                                             # iteration: 8 and 4 iterations per group)
                                             (12288, 512, True), (18944, 256, False),
                                             (8192, 384, True), (256, 96, True)])
def test_swiglu_xq_writes_the_table_of_its_output(orc, wk, in_f, inter, norm):
    qw = wk.DeviceBuffer(2 * inter * in_f // 8, np.uint32)
    si = wk.DeviceBuffer(2 * inter * in_f // 32, np.uint8)
    sb = wk.DeviceBuffer(2 * inter, np.uint32)
    ffi.call("wst_fixture_pack_hier", qw.ptr, si.ptr, sb.ptr, in_f, 0, 2 * inter, 0, 62, 0.02)
    rng = np.random.default_rng(inter)
    x = (rng.standard_normal(in_f) * 3).astype(np.float32)
    nw = dev_f16(wk, f16(orc, 1.0 + 0.1 * rng.standard_normal(in_f).astype(np.float32)))
    src = wk.DeviceBuffer.from_array(x) if norm else dev_f16(wk, f16(orc, x))
    a1, a2 = wk.DeviceBuffer(inter, np.float16), wk.DeviceBuffer(inter, np.float16)
    ffi.call("wst_gemv_hier_swiglu", qw.ptr, si.ptr, sb.ptr, src.ptr, nw.ptr if norm else None,
             np.float32(1e-6), a1.ptr, in_f, inter)
    t2 = wk.DeviceBuffer(inter // 32 * WORDS, np.uint32)
    ffi.call("wst_gemv_hier_swiglu_xq", qw.ptr, si.ptr, sb.ptr, src.ptr, nw.ptr if norm else None,
             np.float32(1e-6), a2.ptr, t2.ptr, in_f, inter)
    assert np.array_equal(a1.numpy().view(np.uint16), a2.numpy().view(np.uint16))
    assert _same_entries(t2.numpy(), _table(wk, a1, inter).numpy())


@pytest.mark.parametrize("n_q,n_kv,hd,max_seq,pos", [(28, 4, 128, 2312, 2100), (14, 2, 64, 1024, 600),
                                                     (28, 4, 128, 8192, 5000)])
def test_attention_xq_writes_the_table_of_its_output(orc, wk, n_q, n_kv, hd, max_seq, pos):
    rng = np.random.default_rng(pos)
    qkv = (rng.standard_normal((n_q + 2 * n_kv) * hd) * 2).astype(np.float32)
    kc = f16(orc, rng.standard_normal(n_kv * max_seq * hd).astype(np.float32)).view(np.float16)
    vc = f16(orc, rng.standard_normal(n_kv * max_seq * hd).astype(np.float32)).view(np.float16)
    rope = wk.RopeTable(max_seq, hd, 1e6)
    cur = wk.DeviceCursor(pos)
    outs, tables = [], []
    for with_table in (False, True):
        c = wk.KvCache(n_kv, n_q, hd, max_seq)
        c.k.copy_from(kc)
        c.v.copy_from(vc)
        q = wk.DeviceBuffer.from_array(qkv)
        o = wk.DeviceBuffer(n_q * hd, np.float16)
        args = (rope.cos.ptr, rope.sin.ptr, c.partials.ptr, o.ptr)
        tail = (n_q, n_kv, hd, cur.buf.ptr, max_seq, np.float32(1.0 / math.sqrt(hd)), None, None,
                np.float32(1e-6))
        if with_table:
            t = wk.DeviceBuffer(n_q * hd // 32 * WORDS, np.uint32)
            ffi.call("wst_attn_decode_fused_xq", q.ptr, c.k.ptr, c.v.ptr, *args, t.ptr, *tail)
            tables.append(t)
        else:
            ffi.call("wst_attn_decode_fused", q.ptr, c.k.ptr, c.v.ptr, *args, *tail)
        outs.append((o, c))
    (o1, c1), (o2, c2) = outs
    assert np.array_equal(o1.numpy().view(np.uint16), o2.numpy().view(np.uint16))
    assert np.array_equal(c1.k.numpy().view(np.uint16), c2.k.numpy().view(np.uint16))
    assert _same_entries(tables[0].numpy(), _table(wk, o1, n_q * hd).numpy())


def test_xq_entry_points_check_their_arguments(wk):
    x = wk.DeviceBuffer(64, np.float16)
    t = wk.DeviceBuffer(2 * WORDS, np.uint32)
    assert ffi.lib().wst_hier_xq_table(x.ptr, t.ptr, 48) != 0
    assert ffi.lib().wst_hier_xq_table(None, t.ptr, 64) != 0
    assert ffi.lib().wst_gemv_hier_swiglu_xq(x.ptr, x.ptr, x.ptr, x.ptr, None, np.float32(1e-6),
                                             x.ptr, t.ptr, 64, 48) != 0


@pytest.mark.parametrize("inter", [96, 160])
def test_swiglu_xq_eight_rows_per_wave_stops_at_the_last_group(orc, wk, monkeypatch, inter):
    """WST_GEMV_RPW=8 (8 rows per wave: 64 rows per block iteration, two table
    groups) with an intermediate size that is a multiple of 32 but not of
    64: the last iteration's second group lies past the output and must not
    be written (a guard entry after the table stays untouched)."""
    monkeypatch.setenv("WST_GEMV_RPW", "8")
    in_f = 896
    qw = wk.DeviceBuffer(2 * inter * in_f // 8, np.uint32)
    si = wk.DeviceBuffer(2 * inter * in_f // 32, np.uint8)
    sb = wk.DeviceBuffer(2 * inter, np.uint32)
    ffi.call("wst_fixture_pack_hier", qw.ptr, si.ptr, sb.ptr, in_f, 0, 2 * inter, 0, 63, 0.02)
    x = np.random.default_rng(inter).standard_normal(in_f).astype(np.float32)
    xd = dev_f16(wk, f16(orc, x))
    a1, a2 = wk.DeviceBuffer(inter, np.float16), wk.DeviceBuffer(inter, np.float16)
    ffi.call("wst_gemv_hier_swiglu", qw.ptr, si.ptr, sb.ptr, xd.ptr, None, np.float32(1e-6),
             a1.ptr, in_f, inter)
    guard = np.full((inter // 32 + 1) * WORDS, 0xA5A5A5A5, np.uint32)
    t2 = wk.DeviceBuffer.from_array(guard)
    ffi.call("wst_gemv_hier_swiglu_xq", qw.ptr, si.ptr, sb.ptr, xd.ptr, None, np.float32(1e-6),
             a2.ptr, t2.ptr, in_f, inter)
    got = t2.numpy()
    assert np.array_equal(a1.numpy().view(np.uint16), a2.numpy().view(np.uint16))
    assert _same_entries(got[:inter // 32 * WORDS], _table(wk, a1, inter).numpy())
    assert np.all(got[inter // 32 * WORDS:] == 0xA5A5A5A5)
