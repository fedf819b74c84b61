"""GPU parity tests of the C ABI kernels against the CPU oracle.

Restates the reference's differential tests
(crates/whetstone-kernels/tests/decode_kernels.rs, rescore_kernels.rs) and adds
the bit-exact checks this backend promises: unpack/embedding, argmax, the
device packer, tile-rule independence, fused == unfused.
"""
import math
import os

import numpy as np
import pytest

from conftest import dev_f16, f16
from whetstone_amd import ffi

pytestmark = pytest.mark.gpu


def _upload_packed(wk, p):
    return wk.QuantLinearHier(p.qw, p.si, p.sb, p.in_f, p.out_f)


def _ref_gemv(orc, p, xbits, bias_bits=None):
    """f64 dot of the oracle's dequantized matrix (hier.rs:398-421) with f16 x,
    computed independently with numpy: y and the scale sum |w x|."""
    w = orc.dequantize(p).astype(np.float64)
    x = orc.f16_value(xbits).astype(np.float64)
    y = w @ x
    if bias_bits is not None:
        y = y + orc.f16_value(bias_bits).astype(np.float64)
    return y, np.abs(w) @ np.abs(x)


# --------------------------------------------------------------------- GEMV

SHAPES_05B = [(896, 1152), (896, 896), (896, 9728), (4864, 896), (896, 4096)]


@pytest.mark.parametrize("in_f,out_f", SHAPES_05B + [(3584, 640), (18944, 96), (1024, 333)])
def test_gemv_matches_dequantized_reference(orc, wk, in_f, out_f):
    """decode_kernels.rs:491-557, with the reference's hash weights and
    RMSNorm-scale activations; tolerance 1e-4 * sum|w x| (the reference allows
    4e-3 for its fp16-accumulating kernel; this one accumulates in f32)."""
    i = np.arange(in_f * out_f, dtype=np.uint64)
    a = ((i * np.uint64(2654435761)) % np.uint64(10000)).astype(np.float32) / 10000.0 - 0.5
    b = ((i * np.uint64(40503)) % np.uint64(977)).astype(np.float32) / 977.0 - 0.5
    w = a * 0.15 + b * b * b * 0.5
    c = np.arange(in_f)
    x = (((c * 7919) % 401).astype(np.float32) / 200.0 - 1.0) * 2.5
    p, _ = orc.quantize(w, in_f, out_f)
    xb = f16(orc, x)
    lin = _upload_packed(wk, p)
    xd = dev_f16(wk, xb)
    yd = wk.DeviceBuffer(out_f, np.float32)
    lin.gemv(xd, yd)
    got = yd.numpy().astype(np.float64)
    want, scale = _ref_gemv(orc, p, xb)
    err = np.abs(got - want) / np.maximum(scale, 1.0)
    assert err.max() < 1e-4, f"{in_f}x{out_f}: worst {err.max():.3g} at row {err.argmax()}"


def test_gemv_bias_and_accumulate(orc, wk):
    in_f, out_f = 896, 1152
    w = orc.fixture_normal(3, 11, in_f * out_f)
    p, _ = orc.quantize(w, in_f, out_f)
    xb = f16(orc, orc.fixture_normal(3, 12, in_f, 1.0))
    bb = f16(orc, orc.fixture_normal(3, 13, out_f, 0.5))
    y0 = orc.fixture_normal(3, 14, out_f, 1.0)
    lin = _upload_packed(wk, p)
    yd = wk.DeviceBuffer.from_array(y0)
    lin.gemv_ex(dev_f16(wk, xb), dev_f16(wk, bb), yd, accumulate=True)
    got = yd.numpy().astype(np.float64)
    want, scale = _ref_gemv(orc, p, xb, bb)
    want = want + y0.astype(np.float64)
    assert np.max(np.abs(got - want) / np.maximum(scale, 1.0)) < 1e-4


def test_tile_rules_agree_bit_for_bit(orc, wk):
    """decode_kernels.rs:560-601 asks 1e-3; here a row's value does not depend
    on the tile at all."""
    in_f, out_f = 896, 1152
    p, _ = orc.quantize(orc.fixture_normal(5, 1, in_f * out_f), in_f, out_f)
    lin = _upload_packed(wk, p)
    xd = dev_f16(wk, f16(orc, orc.fixture_normal(5, 2, in_f, 1.0)))
    saved = wk.hier_get_rule()
    try:
        outs = []
        for t in range(4):
            wk.hier_set_rule(t, t, t)
            yd = wk.DeviceBuffer(out_f, np.float32)
            lin.gemv(xd, yd)
            outs.append(yd.numpy())
        for o in outs[1:]:
            assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))
    finally:
        wk.hier_set_rule(*saved)


def test_gemv_refuses_bad_shapes(orc, wk):
    from whetstone_amd import ffi
    with pytest.raises(wk.ShapeError):
        wk.QuantLinearHier(np.zeros(10, np.uint32), np.zeros(1, np.uint8),
                           np.zeros(1, np.uint32), 100, 1)
    st = ffi.lib().wst_gemv_int4_hier_ex(None, None, None, None, None, None, 32, 1, 0)
    assert st == ffi.WST_ERR_INVALID_ARG


# ---------------------------------------------------------------- embedding


@pytest.mark.parametrize("in_f", [896, 3584])
def test_embedding_row_is_bit_exact(orc, wk, in_f):
    vocab = 300
    p, _ = orc.quantize(orc.fixture_normal(9, 1, in_f * vocab), in_f, vocab)
    lin = _upload_packed(wk, p)
    deq = orc.dequantize(p)
    out = wk.DeviceBuffer(in_f, np.float32)
    for tok, row in [(0, 0), (157, 157), (vocab - 1, vocab - 1), (-5, 0), (10 ** 6, vocab - 1)]:
        cur = wk.DeviceCursor(tok)
        lin.gather_row(cur, out)
        assert np.array_equal(out.numpy().view(np.uint32), deq[row].view(np.uint32)), tok


def test_embedding_chunk_matches_single_rows(orc, wk):
    in_f, vocab, n = 896, 200, 7
    p, _ = orc.quantize(orc.fixture_normal(9, 2, in_f * vocab), in_f, vocab)
    lin = _upload_packed(wk, p)
    toks = np.array([3, 199, 0, 42, 42, 7, 100], np.int32)
    out = wk.DeviceBuffer(n * in_f, np.float32)
    lin.gather_rows(wk.DeviceBuffer.from_array(toks), out, n)
    deq = orc.dequantize(p)
    assert np.array_equal(out.numpy().reshape(n, in_f).view(np.uint32), deq[toks].view(np.uint32))


# ------------------------------------------------------------- decode layers


def test_rmsnorm_matches_reference(orc, wk):
    """decode_kernels.rs:31-58 (f64 reference, tol 2e-3)."""
    n = 896
    i = np.arange(n)
    x = (((i * 37) % 211) / 211.0 - 0.5).astype(np.float32) * 3.0
    w = (0.5 + (i % 17) / 34.0).astype(np.float32)
    wb = f16(orc, w)
    out = wk.DeviceBuffer(n, np.float16)
    wk.rmsnorm(wk.DeviceBuffer.from_array(x), dev_f16(wk, wb), out, 1e-6)
    got = out.numpy().astype(np.float64)
    inv = 1.0 / math.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6)
    want = x.astype(np.float64) * inv * orc.f16_value(wb)
    assert np.all(np.abs(got - want) < 2e-3 * np.maximum(np.abs(want), 1.0))
    # and within one f16 rounding of the oracle
    ob = orc.rmsnorm(x, wb, 1e-6)
    assert np.max(np.abs(got - orc.f16_value(ob))) <= 2e-3


def test_swiglu_matches_reference(orc, wk):
    n = 4864
    i = np.arange(n)
    g = ((i % 97) / 24.0 - 2.0).astype(np.float32)
    u = ((i % 53) / 26.0 - 1.0).astype(np.float32)
    out = wk.DeviceBuffer(n, np.float16)
    wk.swiglu(wk.DeviceBuffer.from_array(np.concatenate([g, u])), out)
    want = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    got = out.numpy().astype(np.float64)
    assert np.all(np.abs(got - want) < 3e-3 * np.maximum(np.abs(want), 1.0))


def _rotate(x, pos, theta):
    hd = x.size
    half = hd // 2
    j = np.arange(half)
    inv = theta ** (-j / half)
    c, s = np.cos(pos * inv), np.sin(pos * inv)
    x1, x2 = x[:half].astype(np.float64), x[half:].astype(np.float64)
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s])


def test_rope_uses_the_half_rotation_layout(orc, wk):
    """decode_kernels.rs:90-126."""
    n_q, n_kv, hd, max_seq, pos, theta = 2, 1, 64, 8, 3, 1e6
    q = ((np.arange(n_q * hd) % 31) / 15.0 - 1.0).astype(np.float32)
    k = ((np.arange(n_kv * hd) % 23) / 11.0 - 1.0).astype(np.float32)
    v = ((np.arange(n_kv * hd) % 19) / 9.0 - 1.0).astype(np.float32)
    table = wk.RopeTable(max_seq, hd, theta)
    cache = wk.KvCache(n_kv, n_q, hd, max_seq)
    qd = wk.DeviceBuffer.from_array(np.concatenate([q, k, v]))
    wk.rope_cache(qd, cache, table, n_q, wk.DeviceCursor(pos))
    got = qd.numpy()
    for h in range(n_q):
        want = _rotate(q[h * hd:(h + 1) * hd], pos, theta)
        assert np.max(np.abs(got[h * hd:(h + 1) * hd] - want)) < 1e-5
    kc = cache.k.numpy().astype(np.float64).reshape(n_kv, max_seq, hd)
    assert np.max(np.abs(kc[0, pos] - _rotate(k, pos, theta))) < 3e-3
    vc = cache.v.numpy().astype(np.float64).reshape(n_kv, max_seq, hd)
    assert np.max(np.abs(vc[0, pos] - v)) < 3e-3


def test_qk_norm_is_per_head_and_precedes_the_rotation(orc, wk):
    """decode_kernels.rs:139-239."""
    n_q, n_kv, hd, max_seq, pos, theta, eps = 4, 2, 64, 8, 5, 1e6, 1e-6
    q = ((np.arange(n_q * hd) % 31) / 15.0 - 1.0).astype(np.float32)
    k = ((np.arange(n_kv * hd) % 23) / 11.0 - 1.0).astype(np.float32)
    v = ((np.arange(n_kv * hd) % 19) / 9.0 - 1.0).astype(np.float32)
    gq = (0.5 + (np.arange(hd) % 7) * 0.1).astype(np.float32)
    gk = (1.5 - (np.arange(hd) % 5) * 0.2).astype(np.float32)
    gqb, gkb = f16(orc, gq), f16(orc, gk)
    table = wk.RopeTable(max_seq, hd, theta)
    cache = wk.KvCache(n_kv, n_q, hd, max_seq)
    qd = wk.DeviceBuffer.from_array(np.concatenate([q, k, v]))
    wk.rope_cache(qd, cache, table, n_q, wk.DeviceCursor(pos),
                  (dev_f16(wk, gqb), dev_f16(wk, gkb), eps))
    got = qd.numpy()

    def norm(x, g):
        x = x.astype(np.float64)
        return x / math.sqrt(np.mean(x * x) + eps) * orc.f16_value(g)

    for h in range(n_q):
        want = _rotate(norm(q[h * hd:(h + 1) * hd], gqb), pos, theta)
        tol = 1e-4 * max(np.max(np.abs(want)), 1.0)
        assert np.max(np.abs(got[h * hd:(h + 1) * hd] - want)) < tol
    kc = cache.k.numpy().astype(np.float64).reshape(n_kv, max_seq, hd)
    vc = cache.v.numpy().astype(np.float64).reshape(n_kv, max_seq, hd)
    for h in range(n_kv):
        want = _rotate(norm(k[h * hd:(h + 1) * hd], gkb), pos, theta)
        assert np.max(np.abs(kc[h, pos] - want)) < 3e-3
        assert np.max(np.abs(vc[h, pos] - v[h * hd:(h + 1) * hd])) < 3e-3


def test_qk_norm_with_unit_gain_on_unit_rms_head_is_identity(orc, wk):
    """decode_kernels.rs:245-287."""
    n_q, n_kv, hd, max_seq, pos = 2, 1, 64, 8, 2
    q = np.where(np.arange(n_q * hd) % 3 == 0, -1.0, 1.0).astype(np.float32)
    k = np.where(np.arange(n_kv * hd) % 5 == 0, -1.0, 1.0).astype(np.float32)
    v = ((np.arange(n_kv * hd) % 19) / 9.0 - 1.0).astype(np.float32)
    ones = dev_f16(wk, f16(orc, np.ones(hd)))
    table = wk.RopeTable(max_seq, hd, 1e6)
    qkv = np.concatenate([q, k, v])
    c1, c2 = wk.KvCache(n_kv, n_q, hd, max_seq), wk.KvCache(n_kv, n_q, hd, max_seq)
    a, b = wk.DeviceBuffer.from_array(qkv), wk.DeviceBuffer.from_array(qkv)
    cur = wk.DeviceCursor(pos)
    wk.rope_cache(a, c1, table, n_q, cur)
    wk.rope_cache(b, c2, table, n_q, cur, (ones, ones, 0.0))
    assert np.max(np.abs(a.numpy() - b.numpy())) < 1e-6


def test_attention_over_one_position_returns_v(orc, wk):
    """decode_kernels.rs:293-329."""
    n_q, n_kv, hd, max_seq = 14, 2, 64, 32
    table = wk.RopeTable(max_seq, hd, 1e6)
    cache = wk.KvCache(n_kv, n_q, hd, max_seq)
    q = ((np.arange(n_q * hd) % 29) / 14.0 - 1.0).astype(np.float32)
    k = ((np.arange(n_kv * hd) % 13) / 6.0 - 1.0).astype(np.float32)
    v = ((np.arange(n_kv * hd) % 17) / 8.0 - 1.0).astype(np.float32)
    qd = wk.DeviceBuffer.from_array(np.concatenate([q, k, v]))
    cur = wk.DeviceCursor(0)
    wk.rope_cache(qd, cache, table, n_q, cur)
    out = wk.DeviceBuffer(n_q * hd, np.float16)
    wk.attn_decode(qd, cache, out, n_q, cur)
    got = out.numpy().astype(np.float32).reshape(n_q, hd)
    vb = orc.f16_value(f16(orc, v)).reshape(n_kv, hd)
    for h in range(n_q):
        assert np.max(np.abs(got[h] - vb[h // (n_q // n_kv)])) < 2e-3


def test_attention_over_two_positions_matches_explicit_softmax(orc, wk):
    """decode_kernels.rs:333-410."""
    n_q, n_kv, hd, max_seq, theta = 2, 1, 64, 16, 1e6
    cache = wk.KvCache(n_kv, n_q, hd, max_seq)
    table = wk.RopeTable(max_seq, hd, theta)
    ks, vs = [], []
    for p in range(2):
        k = (((np.arange(hd) + 7 * p) % 11) / 5.0 - 1.0).astype(np.float32)
        v = (((np.arange(hd) + 3 * p) % 7) / 3.0 - 1.0).astype(np.float32)
        qd = wk.DeviceBuffer.from_array(np.concatenate([np.zeros(n_q * hd, np.float32), k, v]))
        wk.rope_cache(qd, cache, table, n_q, wk.DeviceCursor(p))
        ks.append(orc.f16_value(f16(orc, _rotate(k, p, theta))).astype(np.float64))
        vs.append(orc.f16_value(f16(orc, v)).astype(np.float64))
    q = ((np.arange(n_q * hd) % 5) / 2.0 - 1.0).astype(np.float32)
    out = wk.DeviceBuffer(n_q * hd, np.float16)
    wk.attn_decode(wk.DeviceBuffer.from_array(q), cache, out, n_q, wk.DeviceCursor(1))
    got = out.numpy().astype(np.float64).reshape(n_q, hd)
    for h in range(n_q):
        s = np.array([q[h * hd:(h + 1) * hd].astype(np.float64) @ ks[p] for p in range(2)])
        s /= math.sqrt(hd)
        e = np.exp(s - s.max())
        want = (e[0] * vs[0] + e[1] * vs[1]) / e.sum()
        assert np.max(np.abs(got[h] - want)) < 3e-3


@pytest.mark.parametrize("n_q,n_kv,hd,max_seq,pos", [(14, 2, 64, 1024, 700), (28, 4, 128, 2304, 2047),
                                                     (8, 8, 128, 64, 63), (7, 1, 64, 5000, 4999),
                                                     (4, 2, 256, 300, 150),
                                                     # more than two merge runs (> 32 slices)
                                                     (28, 4, 128, 4608, 4500),
                                                     (14, 2, 64, 9000, 8999),
                                                     # few live slices of many
                                                     (28, 4, 128, 8192, 300),
                                                     # 313 slices of 128 (three merge batches)
                                                     (28, 4, 128, 40000, 39000),
                                                     # 256-dim heads in 32-position slices
                                                     (4, 2, 256, 5000, 4321)])
def test_attention_matches_oracle_on_random_caches(orc, wk, n_q, n_kv, hd, max_seq, pos):
    rng = np.random.default_rng(pos)
    kc = f16(orc, rng.standard_normal(n_kv * max_seq * hd).astype(np.float32))
    vc = f16(orc, rng.standard_normal(n_kv * max_seq * hd).astype(np.float32))
    q = (rng.standard_normal(n_q * hd) * 2).astype(np.float32)
    cache = wk.KvCache(n_kv, n_q, hd, max_seq)
    cache.k.copy_from(kc.view(np.float16))
    cache.v.copy_from(vc.view(np.float16))
    out = wk.DeviceBuffer(n_q * hd, np.float16)
    wk.attn_decode(wk.DeviceBuffer.from_array(q), cache, out, n_q, wk.DeviceCursor(pos))
    want = np.empty(n_q * hd, np.uint16)
    orc.lib().orc_attn_decode(q, kc, vc, want, n_q, n_kv, hd, pos, max_seq,
                              np.float32(1.0 / math.sqrt(hd)))
    got = out.numpy().astype(np.float64)
    assert np.max(np.abs(got - orc.f16_value(want))) < 2e-3


# ------------------------------------------------------------------ argmax


def test_argmax_is_exact_and_ties_go_low(wk):
    """decode_kernels.rs:412-432."""
    n = 151936
    v = np.full(n, -1.0, np.float32)
    v[98765] = 7.5
    idx = wk.DeviceBuffer(1, np.int32)
    wk.argmax(wk.DeviceBuffer.from_array(v), idx)
    assert idx.numpy()[0] == 98765
    v[12345] = 7.5
    wk.argmax(wk.DeviceBuffer.from_array(v), idx)
    assert idx.numpy()[0] == 12345


def test_negative_logits_are_ordered(wk):
    """decode_kernels.rs:462-476."""
    v = (-1.0 - np.arange(4096) * 0.01).astype(np.float32)
    idx = wk.DeviceBuffer(1, np.int32)
    wk.argmax(wk.DeviceBuffer.from_array(v), idx)
    assert idx.numpy()[0] == 0


@pytest.mark.parametrize("n", [1, 7, 1000, 151936, 152064, 300001])
def test_argmax_equals_oracle_key_argmax(orc, wk, n):
    rng = np.random.default_rng(n)
    v = rng.standard_normal(n).astype(np.float32)
    if n > 10:
        v[rng.integers(0, n, 3)] = v.max()  # planted ties
        v[5] = np.inf
        v[6] = -np.inf
        v[7] = -0.0
    idx = wk.DeviceBuffer(1, np.int32)
    for _ in range(3):  # repeated launches reuse the self-resetting counter
        wk.argmax(wk.DeviceBuffer.from_array(v), idx)
        assert idx.numpy()[0] == orc.argmax(v)


@pytest.mark.parametrize("vocab,n", [(151936, 5), (152064, 3), (1001, 4), (8, 2), (40000, 1)])
def test_argmax_rows_equals_oracle_key_argmax(orc, wk, vocab, n):
    """wst_argmax_chunk, a row per token (chunk_ops.cu:425-468): every row's
    pick equals the oracle's key argmax (ties to the lowest index, the
    special values ordered as the single-row argmax orders them). Vocab sizes
    that are a multiple of 4 take the 16-byte-load form, 1001 the scalar one;
    the last row starts 4 bytes off a 16-byte boundary when vocab is odd."""
    rng = np.random.default_rng(vocab + n)
    v = rng.standard_normal(n * vocab).astype(np.float32).reshape(n, vocab)
    if vocab > 10:
        for r in range(n):
            v[r, rng.integers(0, vocab, 3)] = v[r].max()  # planted ties
        v[0, 5] = np.inf
        v[0, 6] = -np.inf
        v[n - 1, vocab - 1] = v[n - 1].max() + 1.0  # the pick in the last 16-byte piece
        if n > 1:
            v[1, :] = -0.0
            v[1, vocab // 2] = 0.0
    d = wk.DeviceBuffer.from_array(v.reshape(-1))
    out = wk.DeviceBuffer(n, np.int32)
    print(f"argmax rows: vocab {vocab} n {n}", flush=True)
    ffi.call("wst_argmax_chunk", d.ptr, out.ptr, vocab, n)
    got = out.numpy()
    for r in range(n):
        assert got[r] == orc.argmax(v[r]), r


def test_nll_matches_host_log_softmax(wk):
    """decode_kernels.rs:434-460."""
    n = 151936
    i = np.arange(n)
    lg = (((i * 7919) % 2003) / 200.0 - 5.0).astype(np.float32)
    acc = wk.DeviceBuffer(2, np.float32)
    d = wk.DeviceBuffer.from_array(lg)
    targets = [0, 1, 12345, 151935]
    for t in targets:
        wk.nll(d, t, acc)
    got = acc.numpy()
    assert int(got[1]) == len(targets)
    m = lg.max().astype(np.float64)
    lse = m + math.log(np.exp(lg.astype(np.float64) - m).sum())
    want = sum(lse - lg[t] for t in targets)
    assert abs(got[0] - want) < 1e-3 * abs(want)


# ----------------------------------------------------------------- rescore


def _rescore_fixture(vocab, hidden):
    i = np.arange(vocab * hidden, dtype=np.uint64)
    head = (((i * np.uint64(2654435761)) % np.uint64(1009)).astype(np.float32) / 504.0 - 1.0)
    x = ((np.arange(hidden) * 40503 % 331) / 165.0 - 1.0).astype(np.float32)
    return head, x


def _exact(orc, head, x, vocab, hidden):
    hb = orc.f16_value(f16(orc, head)).astype(np.float64).reshape(vocab, hidden)
    xb = orc.f16_value(f16(orc, x)).astype(np.float64)
    return (hb @ xb).astype(np.float32)


def test_rescored_rows_match_fp16_reference(orc, wk):
    """rescore_kernels.rs:49-100."""
    vocab, hidden, k = 4096, 256, 64
    head, x = _rescore_fixture(vocab, hidden)
    exact = _exact(orc, head, x, vocab, hidden)
    approx = (exact + ((np.arange(vocab) % 17) - 8.0) * 0.02).astype(np.float32)
    logits = wk.DeviceBuffer.from_array(approx)
    rs = wk.HeadRescore(dev_f16(wk, f16(orc, head)), vocab, hidden, k)
    rs.apply(logits, dev_f16(wk, f16(orc, x)))
    got = logits.numpy()
    count, thresh = rs.last_count(), rs.last_threshold()
    assert count >= k
    o_thresh, o_count, _ = orc.head_threshold(approx, k, rs.cap)
    assert thresh == o_thresh and count == o_count
    sel = approx >= thresh
    assert np.all(np.abs(got[sel] - exact[sel]) < 1e-3 * np.maximum(np.abs(exact[sel]), 1.0))
    assert np.array_equal(got[~sel], approx[~sel])


def test_rescore_restores_the_fp16_argmax(orc, wk):
    """rescore_kernels.rs:106-138."""
    vocab, hidden, k = 8192, 128, 32
    head, x = _rescore_fixture(vocab, hidden)
    exact = _exact(orc, head, x, vocab, hidden)
    approx = (exact + (((np.arange(vocab) * 7919) % 101) - 50.0) * 0.01).astype(np.float32)
    assert int(np.argmax(approx)) != int(np.argmax(exact))
    logits = wk.DeviceBuffer.from_array(approx)
    rs = wk.HeadRescore(dev_f16(wk, f16(orc, head)), vocab, hidden, k)
    rs.apply(logits, dev_f16(wk, f16(orc, x)))
    assert int(np.argmax(logits.numpy())) == int(np.argmax(exact))


def test_threshold_adapts_to_spread(orc, wk):
    """rescore_kernels.rs:143-167."""
    vocab, hidden, k = 4096, 64, 64
    head, x = _rescore_fixture(vocab, hidden)
    hd = dev_f16(wk, f16(orc, head))
    xd = dev_f16(wk, f16(orc, x))
    for spread in (40.0, 0.05):
        lg = (-(np.arange(vocab) % 512) * spread / 512.0).astype(np.float32)
        rs = wk.HeadRescore(hd, vocab, hidden, k)
        rs.apply(wk.DeviceBuffer.from_array(lg), xd)
        assert k <= rs.last_count() < vocab
        assert (rs.last_threshold(), rs.last_count()) == orc.head_threshold(lg, k, rs.cap)[:2]


def test_rescore_refuses_mismatched_shapes(orc, wk):
    """rescore_kernels.rs:170-189."""
    vocab, hidden = 512, 64
    head, x = _rescore_fixture(vocab, hidden)
    hb = dev_f16(wk, f16(orc, head))
    with pytest.raises(wk.ShapeError):
        wk.HeadRescore(hb, vocab, hidden + 1, 8)
    with pytest.raises(wk.ShapeError):
        wk.HeadRescore(hb, vocab, hidden, 0)
    rs = wk.HeadRescore(hb, vocab, hidden, 8)
    with pytest.raises(wk.ShapeError):
        rs.apply(wk.DeviceBuffer(vocab + 1, np.float32), dev_f16(wk, f16(orc, x)))
    with pytest.raises(wk.ShapeError):
        rs.apply(wk.DeviceBuffer(vocab, np.float32), wk.DeviceBuffer(hidden - 1, np.float16))


@pytest.mark.parametrize("in_f,out_f,n,accum", [(896, 1152, 256, False), (3584, 520, 37, True),
                                               (4864, 96, 130, False), (64, 9, 1, True),
                                               (896, 33000, 300, True)])
def test_gemm_int4_hier_matches_dequantised_matmul(orc, wk, in_f, out_f, n, accum):
    """The MFMA chunk GEMM (f16 weight tiles, f32 accumulate) against float64
    dequant(W) @ x. Each weight is rounded to f16 once, so every output is
    within 2^-11 * sum_c |w x| of the exact product (bound used with a 2x
    margin); the bias adds, accumulate adds onto y."""
    w = orc.fixture_normal(6, 1, in_f * out_f)
    p, _ = orc.quantize(w, in_f, out_f)
    lin = wk.QuantLinearHier.from_packed(p)
    wd = orc.dequantize(p).astype(np.float64)  # [out_f][in_f], the quantiser's dequant
    xb = f16(orc, orc.fixture_normal(6, 2, n * in_f, 1.5))
    xf = xb.view(np.float16).astype(np.float64).reshape(n, in_f)
    bias = f16(orc, orc.fixture_normal(6, 3, out_f, 0.3))
    y0 = orc.fixture_normal(6, 4, n * out_f, 1.0).reshape(n, out_f)
    y = wk.DeviceBuffer.from_array(y0.copy())
    xd, bd = dev_f16(wk, xb), dev_f16(wk, bias)  # held: the launch is asynchronous
    ffi.call("wst_gemm_int4_hier", lin.qw.ptr, lin.si.ptr, lin.sb.ptr, xd.ptr, bd.ptr, y.ptr,
             in_f, out_f, n, int(accum))
    got = y.numpy().reshape(n, out_f).astype(np.float64)
    want = xf @ wd.T + bias.view(np.float16).astype(np.float64)
    if accum:
        want += y0
    bound = 2.0 * 2.0 ** -11 * (np.abs(xf) @ np.abs(wd).T) + 1e-5 * (1 + np.abs(want))
    assert np.all(np.abs(got - want) <= bound), float(np.max(np.abs(got - want) / bound))


@pytest.mark.parametrize("in_f,out_f,n", [(896, 200, 256), (128, 64, 3), (40, 17, 5)])
def test_gemm_fp16_matches_matmul(orc, wk, in_f, out_f, n):
    """wst_gemm_fp16 (MFMA for whole 32-column steps, GEMV loop otherwise):
    f16 weights and activations are exact inputs, so only f32 accumulation
    differs from float64."""
    wb = f16(orc, orc.fixture_normal(7, 1, in_f * out_f, 0.05))
    xb = f16(orc, orc.fixture_normal(7, 2, n * in_f, 1.0))
    y = wk.DeviceBuffer(n * out_f, np.float32)
    wd_, xd = dev_f16(wk, wb), dev_f16(wk, xb)  # held: the launch is asynchronous
    ffi.call("wst_gemm_fp16", wd_.ptr, xd.ptr, None, y.ptr, in_f, out_f, n, 0)
    wf = wb.view(np.float16).astype(np.float64).reshape(out_f, in_f)
    xf = xb.view(np.float16).astype(np.float64).reshape(n, in_f)
    want = xf @ wf.T
    got = y.numpy().reshape(n, out_f).astype(np.float64)
    bound = 1e-5 * (np.abs(xf) @ np.abs(wf).T) + 1e-6
    assert np.all(np.abs(got - want) <= bound)


def _with_tg(tg, fn):
    """Runs fn with the chunk attention's token groups per wave forced (1 or
    2; None: the library's choice by token count)."""
    if tg is None:
        return fn()
    os.environ["WST_ATTN_CHUNK_TG"] = str(tg)
    try:
        return fn()
    finally:
        os.environ.pop("WST_ATTN_CHUNK_TG", None)


@pytest.mark.parametrize("tg", [1, 2])
@pytest.mark.parametrize("n_q,n_kv,hd,pos0,n,max_seq", [
    (14, 2, 64, 0, 256, 256), (14, 2, 64, 1000, 44, 1100), (28, 4, 128, 0, 256, 300),
    (28, 4, 128, 3840, 256, 4096), (8, 8, 128, 5, 1, 16), (7, 1, 64, 2000, 37, 2100)])
def test_chunk_attention_equals_per_token_decode_attention(orc, wk, n_q, n_kv, hd, pos0, n,
                                                           max_seq, tg):
    """Chunk attention (chunk_ops.cu:187-265) is decode attention per token:
    token j attends to cache positions [0, pos0 + j] (chunk_kernels.rs:262-360).
    Both token groupings of the MFMA kernel (16 or 32 tokens per block)."""
    rng = np.random.default_rng(pos0 + n + hd)
    kc = f16(orc, rng.standard_normal(n_kv * max_seq * hd).astype(np.float32))
    vc = f16(orc, rng.standard_normal(n_kv * max_seq * hd).astype(np.float32))
    row = (n_q + 2 * n_kv) * hd
    qkv = (rng.standard_normal(n * row) * 2).astype(np.float32)
    cache = wk.KvCache(n_kv, n_q, hd, max_seq)
    cache.k.copy_from(kc.view(np.float16))
    cache.v.copy_from(vc.view(np.float16))
    qd = wk.DeviceBuffer.from_array(qkv)
    out = wk.DeviceBuffer(n * n_q * hd, np.float16)
    scale = np.float32(1.0 / math.sqrt(hd))
    _with_tg(tg, lambda: ffi.call("wst_attn_chunk", qd.ptr, cache.k.ptr, cache.v.ptr, out.ptr,
                                  n_q, n_kv, hd, pos0, n, max_seq, scale))
    got = out.numpy().astype(np.float64).reshape(n, n_q * hd)
    for j in range(n):
        want = np.empty(n_q * hd, np.uint16)
        q = np.ascontiguousarray(qkv[j * row:j * row + n_q * hd])
        orc.lib().orc_attn_decode(q, kc, vc, want, n_q, n_kv, hd, pos0 + j, max_seq, scale)
        assert np.max(np.abs(got[j] - orc.f16_value(want))) < 2e-3, j


@pytest.mark.parametrize("tg", [1, 2])
@pytest.mark.parametrize("n_q,n_kv,hd,pos0,n,max_seq", [
    (14, 2, 64, 0, 256, 300), (28, 4, 128, 1000, 44, 1100), (14, 2, 64, 45, 256, 301),
    (28, 4, 128, 7, 20, 61)])
def test_chunk_attention_ignores_nonfinite_past_the_attended_end(orc, wk, n_q, n_kv, hd, pos0,
                                                                n, max_seq, tg):
    """Cache positions at or past the chunk's last attended position hold NaN
    and Inf (inside the allocation): the output stays finite and equal to
    decode attention, so no tile reads them (a read would give 0 * NaN = NaN
    in P.V). Capacities that are not a multiple of the 32-position tile put
    the last tile past the allocation's end as well."""
    rng = np.random.default_rng(pos0 + n + max_seq)
    kend = min(pos0 + n, max_seq)
    kc = f16(orc, rng.standard_normal(n_kv * max_seq * hd).astype(np.float32))
    vc = f16(orc, rng.standard_normal(n_kv * max_seq * hd).astype(np.float32))
    bad = np.where(np.arange((max_seq - kend) * hd) % 2 == 0, 0x7E00, 0x7C00).astype(np.uint16)
    for c in (kc, vc):
        c3 = c.reshape(n_kv, max_seq, hd)
        c3[:, kend:, :] = bad.reshape(max_seq - kend, hd)
    row = (n_q + 2 * n_kv) * hd
    qkv = (rng.standard_normal(n * row) * 2).astype(np.float32)
    cache = wk.KvCache(n_kv, n_q, hd, max_seq)
    cache.k.copy_from(kc.view(np.float16))
    cache.v.copy_from(vc.view(np.float16))
    qd = wk.DeviceBuffer.from_array(qkv)
    out = wk.DeviceBuffer(n * n_q * hd, np.float16)
    scale = np.float32(1.0 / math.sqrt(hd))
    print(f"chunk attention with NaN/Inf past position {kend}: n_q {n_q} hd {hd} pos0 {pos0} "
          f"n {n} max_seq {max_seq} tg {tg}", flush=True)
    _with_tg(tg, lambda: ffi.call("wst_attn_chunk", qd.ptr, cache.k.ptr, cache.v.ptr, out.ptr,
                                  n_q, n_kv, hd, pos0, n, max_seq, scale))
    got = out.numpy().astype(np.float64).reshape(n, n_q * hd)
    assert np.all(np.isfinite(got))
    for j in range(n):
        want = np.empty(n_q * hd, np.uint16)
        q = np.ascontiguousarray(qkv[j * row:j * row + n_q * hd])
        orc.lib().orc_attn_decode(q, kc, vc, want, n_q, n_kv, hd, pos0 + j, max_seq, scale)
        assert np.max(np.abs(got[j] - orc.f16_value(want))) < 2e-3, j



@pytest.mark.parametrize("n_q,n_kv,hd,pos0,n", [(14, 2, 64, 0, 1536), (28, 4, 128, 300, 700),
                                               (7, 1, 64, 33, 517)])
def test_chunk_attention_token_groupings_are_bit_identical(orc, wk, n_q, n_kv, hd, pos0, n):
    """A token's output does not depend on how many tokens share its block
    (16 or 32): its valid keys are in the same tiles, taken by the same wave in
    the same order, and a block's extra tiles are wholly masked for it. So the
    library may pick the grouping by token count (a batched prefill and the
    same chunks one by one get the same bits). Long prompts (the default picks
    32 here) also checked against decode attention on a sample of tokens."""
    max_seq = pos0 + n + 9
    rng = np.random.default_rng(n + hd)
    kc = f16(orc, rng.standard_normal(n_kv * max_seq * hd).astype(np.float32))
    vc = f16(orc, rng.standard_normal(n_kv * max_seq * hd).astype(np.float32))
    row = (n_q + 2 * n_kv) * hd
    qkv = (rng.standard_normal(n * row) * 2).astype(np.float32)
    cache = wk.KvCache(n_kv, n_q, hd, max_seq)
    cache.k.copy_from(kc.view(np.float16))
    cache.v.copy_from(vc.view(np.float16))
    qd = wk.DeviceBuffer.from_array(qkv)
    scale = np.float32(1.0 / math.sqrt(hd))
    outs = {}
    for tg in (1, 2, None):
        out = wk.DeviceBuffer(n * n_q * hd, np.float16)
        print(f"chunk attention tg {tg}: n_q {n_q} hd {hd} pos0 {pos0} n {n}", flush=True)
        _with_tg(tg, lambda: ffi.call("wst_attn_chunk", qd.ptr, cache.k.ptr, cache.v.ptr,
                                      out.ptr, n_q, n_kv, hd, pos0, n, max_seq, scale))
        outs[tg] = out.numpy().view(np.uint16).copy()
    assert np.array_equal(outs[1], outs[2]), int(np.sum(outs[1] != outs[2]))
    assert np.array_equal(outs[None], outs[2])
    got = outs[2].view(np.float16).astype(np.float64).reshape(n, n_q * hd)
    for j in sorted({0, 1, 31, 32, n // 2, n - 33, n - 1}):
        want = np.empty(n_q * hd, np.uint16)
        q = np.ascontiguousarray(qkv[j * row:j * row + n_q * hd])
        orc.lib().orc_attn_decode(q, kc, vc, want, n_q, n_kv, hd, pos0 + j, max_seq, scale)
        assert np.max(np.abs(got[j] - orc.f16_value(want))) < 2e-3, j