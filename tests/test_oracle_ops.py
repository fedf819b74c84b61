"""Pins the oracle's decode ops against closed forms and the reference's own
kernel tests, restated (crates/whetstone-kernels/tests/decode_kernels.rs,
rescore_kernels.rs). CPU only."""
import math

import numpy as np
import pytest


def _f16(orc, x):
    return orc.f16_bits(np.asarray(x, np.float32))


def _val(orc, bits):
    return orc.f16_value(bits).astype(np.float64)


def _ulp16(v):
    """One f16 ulp at |v| (subnormal floor 2^-24). Checks allow half an ulp
    plus 2^-10 of it: the oracle narrows f64 -> f32 -> f16 like the kernels,
    and the double rounding may land a hair past the halfway point."""
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0**-14)))
    return 2.0 ** (e - 10)


# ------------------------------------------------------------------ GEMV

@pytest.mark.parametrize("in_f,out_f", [(896, 1152), (896, 896), (896, 9728), (4864, 896),
                                        (896, 4096)])
def test_gemv_matches_dequant_times_x(orc, in_f, out_f):
    """decode_kernels.rs:491-557 shapes; y = dequant(W) @ f16(x) (+ bias),
    compared with numpy's float64 matmul at f32 resolution."""
    rng = np.random.default_rng(in_f + out_f)
    w = (rng.standard_normal(in_f * out_f) * 0.02).astype(np.float32)
    p, _ = orc.quantize(w, in_f, out_f)
    xb = _f16(orc, rng.standard_normal(in_f))
    bias = _f16(orc, rng.standard_normal(out_f) * 0.1)
    wd = orc.dequantize(p).astype(np.float64)
    want = wd @ _val(orc, xb) + _val(orc, bias)
    got = orc.gemv(p, xb, bias)
    scale = np.abs(wd) @ np.abs(_val(orc, xb))
    assert np.all(np.abs(got - want) <= 1e-6 * scale + 1e-7)
    acc = rng.standard_normal(out_f).astype(np.float32)
    got2 = orc.gemv(p, xb, None, acc, accum=True)
    assert np.all(np.abs(got2 - (acc + wd @ _val(orc, xb))) <= 1e-6 * (scale + np.abs(acc)) + 1e-6)


def test_gemv_fp16_matches_numpy(orc):
    rng = np.random.default_rng(5)
    in_f, out_f = 256, 64
    wb = _f16(orc, rng.standard_normal(in_f * out_f) * 0.05)
    xb = _f16(orc, rng.standard_normal(in_f))
    y = np.zeros(out_f, np.float32)
    orc.lib().orc_gemv_fp16(wb, xb, None, y, in_f, out_f, 0)
    want = _val(orc, wb).reshape(out_f, in_f) @ _val(orc, xb)
    assert np.max(np.abs(y - want)) < 1e-5


# --------------------------------------------------- rmsnorm and swiglu

def test_rmsnorm_closed_form(orc):
    """decode_kernels.rs:31-58 (f64 reference)."""
    rng = np.random.default_rng(1)
    n = 896
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    wb = _f16(orc, 1 + rng.standard_normal(n) * 0.1)
    got = _val(orc, orc.rmsnorm(x, wb, 1e-6))
    want = x / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * _val(orc, wb)
    assert np.all(np.abs(got - want) <= 0.5 * (1 + 2**-10) * _ulp16(want) + 1e-12)


def test_swiglu_closed_form(orc):
    """decode_kernels.rs:60-85: out = f16(silu(g) * u)."""
    rng = np.random.default_rng(2)
    n = 4864
    gu = (rng.standard_normal(2 * n) * 4).astype(np.float32)
    out = np.empty(n, np.uint16)
    orc.lib().orc_swiglu(gu, out, n)
    g, u = gu[:n].astype(np.float64), gu[n:].astype(np.float64)
    want = g / (1 + np.exp(-g)) * u
    assert np.all(np.abs(_val(orc, out) - want) <= 0.5 * (1 + 2**-10) * _ulp16(want) + 1e-12)


# -------------------------------------------------------------- RoPE

def test_rope_table_closed_form(orc):
    """decode.rs:95-147: invf = theta^(-j/half) in f64, angle in f64, f32 out."""
    max_seq, hd, theta = 300, 128, 1e6
    c, s = orc.rope_table(max_seq, hd, theta)
    half = hd // 2
    p = np.arange(max_seq, dtype=np.float64)[:, None]
    a = p * theta ** (-np.arange(half, dtype=np.float64) / half)[None, :]
    assert np.max(np.abs(c.reshape(max_seq, half) - np.cos(a))) < 6e-8
    assert np.max(np.abs(s.reshape(max_seq, half) - np.sin(a))) < 6e-8


def _rope_call(orc, qkv, n_q, n_kv, hd, pos, max_seq, qn=None, kn=None, eps=1e-6):
    c, s = orc.rope_table(max_seq, hd, 1e6)
    kc = np.zeros(n_kv * max_seq * hd, np.uint16)
    vc = np.zeros_like(kc)
    q = qkv.copy()
    orc.lib().orc_rope_cache(q, kc, vc, c, s, n_q, n_kv, hd, pos, max_seq,
                             None if qn is None else qn.ctypes.data,
                             None if kn is None else kn.ctypes.data, eps)
    return q, kc.reshape(n_kv, max_seq, hd), vc.reshape(n_kv, max_seq, hd), c, s


def test_rope_half_rotation(orc):
    """decode_kernels.rs:90-126: (x1 c - x2 s, x2 c + x1 s), j paired with j+hd/2."""
    rng = np.random.default_rng(3)
    n_q, n_kv, hd, pos, max_seq = 4, 2, 64, 37, 64
    qkv = rng.standard_normal((n_q + 2 * n_kv) * hd).astype(np.float32)
    q, kc, vc, c, s = _rope_call(orc, qkv, n_q, n_kv, hd, pos, max_seq)
    half = hd // 2
    a = pos * 1e6 ** (-np.arange(half) / half)
    cc, ss = np.cos(a), np.sin(a)
    x = qkv.astype(np.float64).reshape(-1, hd)
    rot = np.concatenate([x[:, :half] * cc - x[:, half:] * ss, x[:, half:] * cc + x[:, :half] * ss], 1)
    assert np.max(np.abs(q.reshape(-1, hd)[:n_q] - rot[:n_q])) < 1e-5
    k = _val(orc, kc[:, pos].ravel()).reshape(n_kv, hd)
    assert np.all(np.abs(k - rot[n_q:n_q + n_kv]) <= _ulp16(rot[n_q:n_q + n_kv]) + 1e-5)
    v = _val(orc, vc[:, pos].ravel()).reshape(n_kv, hd)
    assert np.all(np.abs(v - x[n_q + n_kv:]) <= 0.5 * _ulp16(x[n_q + n_kv:]) + 1e-12)
    assert not kc[:, :pos].any() and not kc[:, pos + 1:].any()  # only slot pos is written


def test_qk_norm_normalises_before_rotation_and_leaves_v(orc):
    """decode_kernels.rs:139-239: per-head RMSNorm with a shared [hd] gain,
    applied to q and k before the rotation; v untouched."""
    rng = np.random.default_rng(4)
    n_q, n_kv, hd, pos, max_seq = 4, 2, 128, 5, 16
    qkv = (rng.standard_normal((n_q + 2 * n_kv) * hd) * 3).astype(np.float32)
    qn = _f16(orc, 1 + rng.standard_normal(hd) * 0.1)
    kn = _f16(orc, 1 + rng.standard_normal(hd) * 0.1)
    q, kc, vc, _, _ = _rope_call(orc, qkv, n_q, n_kv, hd, pos, max_seq, qn, kn)
    x = qkv.astype(np.float64).reshape(-1, hd)
    g = np.where(np.arange(n_q + 2 * n_kv)[:, None] < n_q, _val(orc, qn), _val(orc, kn))
    xn = x / np.sqrt(np.mean(x**2, axis=1, keepdims=True) + 1e-6) * g
    half = hd // 2
    a = pos * 1e6 ** (-np.arange(half) / half)
    rot = np.concatenate([xn[:, :half] * np.cos(a) - xn[:, half:] * np.sin(a),
                          xn[:, half:] * np.cos(a) + xn[:, :half] * np.sin(a)], 1)
    assert np.max(np.abs(q.reshape(-1, hd)[:n_q] - rot[:n_q])) < 1e-5
    v = _val(orc, vc[:, pos].ravel()).reshape(n_kv, hd)
    assert np.all(np.abs(v - x[n_q + n_kv:]) <= 0.5 * _ulp16(x[n_q + n_kv:]) + 1e-12)


def test_unit_gain_on_unit_rms_head_equals_no_norm(orc):
    """decode_kernels.rs:245-287."""
    rng = np.random.default_rng(6)
    n_q, n_kv, hd, pos, max_seq = 2, 1, 64, 9, 16
    x = rng.standard_normal(((n_q + 2 * n_kv), hd))
    x = x / np.sqrt(np.mean(x**2, axis=1, keepdims=True))
    qkv = x.astype(np.float32).ravel()
    one = _f16(orc, np.ones(hd))
    a = _rope_call(orc, qkv, n_q, n_kv, hd, pos, max_seq, one, one, eps=0.0)
    b = _rope_call(orc, qkv, n_q, n_kv, hd, pos, max_seq)
    assert np.max(np.abs(a[0] - b[0])) < 1e-5
    assert np.max(np.abs(_val(orc, a[1].ravel()) - _val(orc, b[1].ravel()))) < 2e-3


# --------------------------------------------------------- attention

def _attn(orc, q, kc, vc, n_q, n_kv, hd, pos, max_seq, scale):
    out = np.zeros(n_q * hd, np.uint16)
    orc.lib().orc_attn_decode(q, kc, vc, out, n_q, n_kv, hd, pos, max_seq, scale)
    return _val(orc, out).reshape(n_q, hd)


def test_attention_one_position_returns_v(orc):
    """decode_kernels.rs:293-329."""
    rng = np.random.default_rng(7)
    n_q, n_kv, hd, max_seq = 4, 2, 64, 8
    q = rng.standard_normal(n_q * hd).astype(np.float32)
    kc = _f16(orc, rng.standard_normal(n_kv * max_seq * hd))
    vc = _f16(orc, rng.standard_normal(n_kv * max_seq * hd))
    out = _attn(orc, q, kc, vc, n_q, n_kv, hd, 0, max_seq, 0.125)
    v0 = _val(orc, vc).reshape(n_kv, max_seq, hd)[:, 0]
    assert np.array_equal(out, v0[np.arange(n_q) // (n_q // n_kv)])


def test_attention_two_positions_equal_explicit_softmax(orc):
    """decode_kernels.rs:333-410, with GQA head -> kv head mapping h / (nq/nkv)."""
    rng = np.random.default_rng(8)
    n_q, n_kv, hd, max_seq, pos = 6, 2, 128, 4, 1
    scale = 1 / math.sqrt(hd)
    q = rng.standard_normal(n_q * hd).astype(np.float32)
    kc = _f16(orc, rng.standard_normal(n_kv * max_seq * hd))
    vc = _f16(orc, rng.standard_normal(n_kv * max_seq * hd))
    out = _attn(orc, q, kc, vc, n_q, n_kv, hd, pos, max_seq, scale)
    K = _val(orc, kc).reshape(n_kv, max_seq, hd)
    V = _val(orc, vc).reshape(n_kv, max_seq, hd)
    for h in range(n_q):
        kv = h // (n_q // n_kv)
        qs = (q[h * hd:(h + 1) * hd] * np.float32(scale)).astype(np.float64)
        s = K[kv, :2] @ qs
        p = np.exp(s - s.max())
        p /= p.sum()
        want = p @ V[kv, :2]
        assert np.all(np.abs(out[h] - want) <= 0.5 * _ulp16(want) + 1e-9)


# ------------------------------------------------------------- argmax

def test_argmax_planted_and_low_index_ties(orc):
    """decode_kernels.rs:412-432."""
    v = np.zeros(151936, np.float32)
    v[77777] = 3.0
    assert orc.argmax(v) == 77777
    v[1234] = 3.0
    assert orc.argmax(v) == 1234  # ties go to the lowest index
    assert orc.argmax(np.zeros(10, np.float32)) == 0


def test_argmax_all_negative_and_special_values(orc):
    """decode_kernels.rs:462-476; +inf beats finite, +NaN beats +inf, +0 beats -0."""
    v = -np.arange(1, 1001, dtype=np.float32)
    v[500] = -0.5
    assert orc.argmax(v) == 500
    v[900] = np.inf
    assert orc.argmax(v) == 900
    v[950] = np.nan
    assert orc.argmax(v) == 950
    assert orc.argmax(np.array([-0.0, 0.0], np.float32)) == 1


def test_argmax_equals_key_maximum(orc):
    rng = np.random.default_rng(9)
    v = rng.standard_normal(5000).astype(np.float32)
    v[rng.integers(0, 5000, 50)] = np.float32(v.max())
    b = v.view(np.uint32).astype(np.uint64)
    key = np.where(b & 0x80000000, ~b & 0xFFFFFFFF, b | 0x80000000)
    assert orc.argmax(v) == int(np.flatnonzero(key == key.max())[0])


# --------------------------------------------------------- head ladder

def test_head_threshold_hand_computed(orc):
    """logits[i] = -i/64: the rung 2^c/64 admits 2^c + 1 rows; the smallest
    rung holding k = 64 is c = 6 (65 rows, threshold max - 1)."""
    v = -(np.arange(4096, dtype=np.float32) / np.float32(64.0))
    t, cnt, rung = orc.head_threshold(v, 64, 1024)
    assert (t, cnt, rung) == (-1.0, 65, 6)
    t, cnt, rung = orc.head_threshold(v, 600, 1024)  # 2^10 + 1 = 1025 > cap: step down
    assert (rung, cnt) == (9, 513)


@pytest.mark.parametrize("spread", [40.0, 0.05], ids=["spiked", "flat"])
def test_head_threshold_adapts_to_spread(orc, spread):
    """rescore_kernels.rs:143-167."""
    vocab, k = 4096, 64
    v = (-(np.arange(vocab) % 512).astype(np.float32) * np.float32(spread) / np.float32(512.0))
    _, cnt, _ = orc.head_threshold(v, k, min(16 * k, vocab))
    assert k <= cnt < vocab


def test_head_rescore_rewrites_only_selected_rows(orc):
    """rescore_kernels.rs:49-100: selected rows equal the f64 fp16 dot."""
    rng = np.random.default_rng(10)
    vocab, hidden = 2048, 128
    head = _f16(orc, rng.standard_normal(vocab * hidden) * 0.05)
    x = _f16(orc, rng.standard_normal(hidden))
    exact = _val(orc, head).reshape(vocab, hidden) @ _val(orc, x)
    approx = (exact + rng.standard_normal(vocab) * 0.01).astype(np.float32)
    t, cnt, _ = orc.head_threshold(approx, 32, 512)
    got = approx.copy()
    orc.lib().orc_head_rescore(head, x, got, vocab, hidden, t)
    sel = approx >= t
    assert sel.sum() == cnt
    assert np.max(np.abs(got[sel] - exact[sel])) < 1e-5
    assert np.array_equal(got[~sel], approx[~sel])
