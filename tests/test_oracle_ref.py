"""Pins the oracle's ORC_ACC_REF mode: the reference CUDA kernels' own arithmetic.

ORC_ACC_REF restates, in oracle/oracle.c, how the reference's kernels round
(f16 `__hadd2`/`__hfma2` group sums in the int4 GEMV, gemv_hier.cu:118-163 and
hier.cuh:24-60; the 32-lane xor butterfly and block reductions,
common.cuh:127-161; RMSNorm, decode.cu:46-100; the split attention with its
per-warp online softmax and split merge, attention.cu:57-237).

Each piece is checked here against an independent step-by-step emulation in
numpy, whose float16 conversion of a float64 rounds to nearest even directly
(one rounding), and whose float32 arithmetic is IEEE. The emulation is a second
implementation of the same sequence, written from the reference kernels, not
from the oracle's C: a dropped rounding, a wrong lane mapping, a swapped
nibble or a different reduction order makes the bits differ. Two closed checks
guard the emulation itself: numpy's f16 rounding against the definition on
every f16 midpoint, and a planted case where one rounding (fma) and two
(multiply, then add) give different f16 results.
"""
import numpy as np
import pytest

from oracle import oracle as O

L = O.lib()


def h16(v):
    """f16 RNE of an exactly representable float64 (one rounding)."""
    return np.float16(np.float64(v))


def fma32(a, b, c):
    """fmaf: the f32 product is exact in f64; the sum is rounded once to f64,
    then to f32 (a double rounding only at f32 ties closer than 2^-29)."""
    return np.float32(np.float64(np.float32(a)) * np.float64(np.float32(b)) + np.float64(np.float32(c)))


def warp_sum(p):
    """warp_reduce_sum's xor butterfly as lane 0 sees it."""
    p = np.array(p, np.float32)
    off = 16
    while off >= 1:
        p[:off] = p[:off] + p[off:2 * off]
        off //= 2
    return np.float32(p[0])


def block_sum(v):
    """block_reduce_sum over len(v) threads (a multiple of 32 or padded)."""
    v = np.asarray(v, np.float32)
    nw = (v.size + 31) // 32
    pad = np.zeros(nw * 32, np.float32)
    pad[:v.size] = v
    ws = [warp_sum(pad[w * 32:(w + 1) * 32]) for w in range(nw)]
    p = np.zeros(32, np.float32)
    p[:nw] = ws
    return warp_sum(p)


def rexp(x):
    return np.float32(np.exp(np.float64(np.float32(x))))


# ------------------------------------------------------------------ rounding

def test_d2h_matches_numpy_rne():
    rng = np.random.default_rng(0)
    mids = (np.arange(0, 0x7BFF, dtype=np.uint16).view(np.float16).astype(np.float64)
            + np.arange(1, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)) / 2
    vals = np.concatenate([
        mids, -mids,
        rng.standard_normal(20000) * np.exp2(rng.integers(-26, 17, 20000)),
        rng.integers(-2 ** 40, 2 ** 40, 20000) * 2.0 ** -24,
        [65504.0, 65519.99, 65520.0, 1e6, -1e6, 2.0 ** -25, 2.0 ** -24 * 1.5, 0.0, -0.0]])
    got = np.array([L.orc_d2h(float(v)) for v in vals], np.uint16)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    # numpy's conversion itself on the midpoints: ties go to the even mantissa
    lo = np.arange(0, 0x7BFF, dtype=np.uint16)
    r = mids.astype(np.float16).view(np.uint16)
    assert np.all((r == lo) | (r == lo + 1))
    assert np.all(r % 2 == 0)


def test_hfma_rounds_once():
    """A planted case: q*x + c rounded once differs from the product rounded to
    f16 first. The oracle's hfma must take the single rounding."""
    rng = np.random.default_rng(1)
    found = 0
    for _ in range(20000):
        q = float(rng.integers(-8, 8))
        x = np.float16(rng.standard_normal())
        c = np.float16(rng.standard_normal() * 4)
        once = h16(q * float(x) + float(c))
        twice = h16(float(h16(q * float(x))) + float(c))
        got = L.orc_ref_hfma(int(np.float16(q).view(np.uint16)), int(x.view(np.uint16)),
                             int(c.view(np.uint16)))
        assert got == int(once.view(np.uint16))
        found += int(once != twice)
    assert found > 0  # the distinction is exercised
    a, b = np.float16(1.0), np.float16(2.0 ** -11)
    assert L.orc_ref_hadd(int(a.view(np.uint16)), int(b.view(np.uint16))) == 0x3C00  # tie to even
    b = np.float16(3 * 2.0 ** -11)
    assert L.orc_ref_hadd(int(a.view(np.uint16)), int(b.view(np.uint16))) == 0x3C02


# ------------------------------------------------------------------ int4 GEMV

def emulate_gemv_row(qw_row, si_row, sbw, x16):
    """gemv_int4_hier_kernel for one row, step by step (gemv_hier.cu:118-163)."""
    d = np.float32(np.uint16(sbw & 0xFFFF).view(np.float16))
    dm = np.float32(np.uint16(sbw >> 16).view(np.float16))
    G = si_row.size
    lanes = np.zeros(32, np.float32)
    for lane in range(32):
        a = np.float32(0)
        for v in range(lane, G, 32):
            xg = x16[32 * v:32 * v + 32]
            xs = [np.float16(0), np.float16(0)]
            for i in range(16):
                for h in range(2):
                    xs[h] = h16(float(xs[h]) + float(xg[2 * i + h]))
            sx = np.float32(xs[0]) + np.float32(xs[1])
            idx = int(si_row[v])
            s = d * np.float32(idx & 15)
            m = -dm * np.float32(idx >> 4)
            dot = [np.float16(0), np.float16(0)]
            for w in range(4):
                word = int(qw_row[4 * v + w])
                for i in range(4):
                    for h in range(2):
                        q = ((word >> (8 * i + 4 * h)) & 15) - 8
                        dot[h] = h16(q * float(xg[8 * w + 2 * i + h]) + float(dot[h]))
            dotf = np.float32(dot[0]) + np.float32(dot[1])
            a = fma32(s, dotf, a)
            a = fma32(fma32(8.0, s, m), sx, a)
        lanes[lane] = a
    return warp_sum(lanes)


@pytest.mark.parametrize("in_f,out_f,xs", [(64, 5, 1.0), (1088, 3, 1.0), (2112, 2, 30.0)])
def test_ref_gemv_matches_emulation(in_f, out_f, xs):
    rng = np.random.default_rng(in_f)
    w = rng.standard_normal((out_f, in_f)).astype(np.float32) * 0.02
    p, _ = O.quantize(w, in_f, out_f)
    x = (rng.standard_normal(in_f) * xs).astype(np.float16)
    bias = rng.standard_normal(out_f).astype(np.float16)
    y0 = rng.standard_normal(out_f).astype(np.float32)
    with O.variant(O.ACC_REF):
        got = O.gemv(p, x.view(np.uint16), bias.view(np.uint16), y0, accum=True)
    qw = p.qw.reshape(out_f, in_f // 8)
    si = p.si.reshape(out_f, in_f // 32)
    for r in range(out_f):
        want = y0[r] + (emulate_gemv_row(qw[r], si[r], int(p.sb[r]), x) + np.float32(bias[r]))
        assert got[r].view(np.uint32) == np.float32(want).view(np.uint32), (r, got[r], want)
    # and it is a dot product: close to float64 (f16 group sums: ~2^-11 relative)
    ref = O.dequantize(p).astype(np.float64) @ x.astype(np.float64) + bias + y0
    scale = np.abs(O.dequantize(p)).astype(np.float64) @ np.abs(x.astype(np.float64))
    assert np.all(np.abs(got - ref) <= 2e-3 * scale + 1e-6)


def test_ref_gemv_differs_from_f64_sum():
    """The mode is not the f64 oracle under another name: on a row long enough
    for f16 group sums to round, the results differ."""
    rng = np.random.default_rng(5)
    w = rng.standard_normal((64, 3584)).astype(np.float32) * 0.02
    p, _ = O.quantize(w, 3584, 64)
    x = rng.standard_normal(3584).astype(np.float16).view(np.uint16)
    a = O.gemv(p, x)
    with O.variant(O.ACC_REF):
        b = O.gemv(p, x)
    assert np.any(a != b)


# ------------------------------------------------------------------ RMSNorm

@pytest.mark.parametrize("n", [896, 3584])
def test_ref_rmsnorm_matches_emulation(n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float16)
    eps = np.float32(1e-6)
    with O.variant(O.ACC_REF):
        got = O.rmsnorm(x, w.view(np.uint16), float(eps))
    if n <= 1024:
        t = np.zeros((n + 31) // 32 * 32, np.float32)
        t[:n] = x * x
    else:
        t = np.zeros(256, np.float32)
        for th in range(256):
            for i in range(th, n, 256):
                t[th] = fma32(x[i], x[i], t[th])
    inv = np.float32(1) / np.sqrt(block_sum(t) / np.float32(n) + eps)
    want = ((x * inv) * w.astype(np.float32)).astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# ------------------------------------------------------------------ attention

def test_ref_attn_splits_formula():
    """pick_splits (attention.cu:201-218): ceil(2*SMs/n_q), at most 16, shrunk
    until every slice holds 8 positions."""
    L.orc_set_ref_sms(30)
    assert L.orc_ref_attn_splits(14, 4096) == 5
    assert L.orc_ref_attn_splits(28, 2312) == 3
    assert L.orc_ref_attn_splits(4, 48) == 6
    L.orc_set_ref_sms(128)
    assert L.orc_ref_attn_splits(14, 4096) == 16
    assert L.orc_ref_attn_splits(14, 40) == 5
    L.orc_set_ref_sms(30)


def emulate_attention(q, kc, vc, n_q, n_kv, hd, seq, max_seq, scale, splits):
    gqa = n_q // n_kv
    epl = hd // 32
    per = (seq + splits - 1) // splits
    out = np.zeros((n_q, hd), np.float16)
    for h in range(n_q):
        kvh = h // gqa
        qs = (q[h] * np.float32(scale)).astype(np.float32)
        parts = []
        for sp in range(splits):
            t0, t1 = sp * per, min(sp * per + per, seq)
            if t0 >= t1:
                parts.append((np.float32(-np.inf), np.float32(0), np.zeros(hd, np.float32)))
                continue
            ms, ls, accs = [], [], []
            for w in range(8):
                m, l = np.float32(-np.inf), np.float32(0)
                acc = np.zeros(hd, np.float32)
                for t in range(t0 + w, t1, 8):
                    k = kc[kvh, t].astype(np.float32)
                    v = vc[kvh, t].astype(np.float32)
                    lanes = np.zeros(32, np.float32)
                    for lane in range(32):
                        a = np.float32(0)
                        for i in range(epl):
                            a = fma32(qs[lane + 32 * i], k[lane + 32 * i], a)
                        lanes[lane] = a
                    s = warp_sum(lanes)
                    m_new = max(m, s)
                    corr, pr = rexp(m - m_new), rexp(s - m_new)
                    acc = np.array([fma32(pr, v[d], acc[d] * corr) for d in range(hd)], np.float32)
                    l = fma32(l, corr, pr)
                    m = m_new
                ms.append(m); ls.append(l); accs.append(acc)
            M = max(ms)
            num = np.zeros(hd, np.float32)
            den = np.float32(0)
            for w in range(8):
                f = rexp(ms[w] - M)
                num = np.array([fma32(accs[w][d], f, num[d]) for d in range(hd)], np.float32)
                den = fma32(ls[w], f, den)
            parts.append((M, den, num))
        M = max(p[0] for p in parts)
        num = np.zeros(hd, np.float32)
        den = np.float32(0)
        for (pm, pl, pn) in parts:
            f = rexp(pm - M)
            num = np.array([fma32(pn[d], f, num[d]) for d in range(hd)], np.float32)
            den = fma32(pl, f, den)
        out[h] = (num / den).astype(np.float16)
    return out


@pytest.mark.parametrize("sms,pos", [(30, 40), (2, 40), (30, 3)])
def test_ref_attention_matches_emulation(sms, pos):
    n_q, n_kv, hd, max_seq = 4, 2, 64, 48
    rng = np.random.default_rng(sms + pos)
    q = (rng.standard_normal((n_q, hd)) * 2).astype(np.float32)
    kc = rng.standard_normal((n_kv, max_seq, hd)).astype(np.float16)
    vc = rng.standard_normal((n_kv, max_seq, hd)).astype(np.float16)
    out = np.zeros((n_q, hd), np.uint16)
    scale = np.float32(1) / np.sqrt(np.float32(hd))
    L.orc_set_ref_sms(sms)
    try:
        with O.variant(O.ACC_REF):
            L.orc_attn_decode(q.ravel(), kc.view(np.uint16).ravel(), vc.view(np.uint16).ravel(),
                              out.ravel(), n_q, n_kv, hd, pos, max_seq, float(scale))
        splits = L.orc_ref_attn_splits(n_q, max_seq)
    finally:
        L.orc_set_ref_sms(30)
    # the out buffer was filled in place through its flat view
    want = emulate_attention(q, kc, vc, n_q, n_kv, hd, pos + 1, max_seq, scale, splits)
    assert np.array_equal(out, want.view(np.uint16))


# ------------------------------------------------------------------ SwiGLU / forward

def test_ref_swiglu_matches_emulation():
    rng = np.random.default_rng(9)
    n = 300
    gu = (rng.standard_normal(2 * n) * 4).astype(np.float32)
    out = np.zeros(n, np.uint16)
    with O.variant(O.ACC_REF):
        L.orc_swiglu(gu, out, n)
    g, u = gu[:n], gu[n:]
    rc = np.float32(1) / (np.float32(1) + np.array([rexp(-v) for v in g], np.float32))
    want = ((g * rc) * u).astype(np.float16).view(np.uint16)
    assert np.array_equal(out, want)


def test_ref_forward_close_to_f64():
    """The whole REF step stays within f16 noise of the f64 oracle at the tiny
    shape, and its argmax stream agrees on non-ties."""
    m = O.Model(O.TINY, 0)
    prompt = np.random.default_rng(1).integers(0, O.TINY["vocab"], 8)
    lgs = {}
    for acc in (O.ACC_F64, O.ACC_REF):
        with O.variant(acc):
            st = O.State(m, 32, 0)
            for t in prompt:
                _, lg = st.step(int(t))
            lgs[acc] = lg.astype(np.float64)
            st.close()
    d = np.max(np.abs(lgs[O.ACC_F64] - lgs[O.ACC_REF]))
    assert 0 < d < 2e-2


def test_ref_gemv_overflowing_group_sum_matches_emulation():
    """x large enough that an f16 group partial overflows to inf: the oracle
    leaves its integer fast path for the f16 one, and still follows the
    kernel (inf enters the row sum; the other rows are unaffected)."""
    in_f, out_f = 64, 4
    rng = np.random.default_rng(11)
    w = rng.standard_normal((out_f, in_f)).astype(np.float32) * 0.02
    p, _ = O.quantize(w, in_f, out_f)
    x = (rng.standard_normal(in_f) * 0.5).astype(np.float16)
    x[3] = np.float16(60000.0)
    x[35] = np.float16(-60000.0)
    with O.variant(O.ACC_REF):
        got = O.gemv(p, x.view(np.uint16))
    qw = p.qw.reshape(out_f, in_f // 8)
    si = p.si.reshape(out_f, in_f // 32)
    with np.errstate(over="ignore", invalid="ignore"):
        for r in range(out_f):
            want = np.float32(emulate_gemv_row(qw[r], si[r], int(p.sb[r]), x))
            if np.isnan(want):
                assert np.isnan(got[r]), (r, got[r])
            else:
                assert got[r].view(np.uint32) == want.view(np.uint32), (r, got[r], want)
    assert not np.all(np.isfinite(got))  # the overflow is exercised
