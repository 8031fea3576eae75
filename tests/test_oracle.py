"""Pins the CPU oracle (oracle/bgl_oracle.c) before any GPU result is compared with it.

Each packer/decoder is checked against (a) the reference's own C sources compiled in place
(oracle/_ref, bit-exact), (b) the reference's known-answer tests and pinned control constants
(tests/regression/*.c, tools/qng64_dense_test.c), and (c) identities the mathematics fixes,
chosen so that a dropped term, wrong sign, wrong index or transposed operand fails."""
import ctypes as C

import numpy as np
import pytest

from golden.fixtures import gate9, kat_qng64, reg_probe, seeded_normal, tiny_st
from oracle_ffi import _ptr, expert_struct

QNG_NS = [2, 3, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15]


def _weights(seed, out, inn, sigma=0.02, outliers=True, zero_rows=True):
    w = seeded_normal(seed, (out, inn), sigma)
    if outliers:
        rng = np.random.default_rng(seed + 1)
        m = rng.random(w.shape) < 0.01
        w[m] *= 8
    if zero_rows and out > 2:
        w[1, :] = 0.0                          # all-zero groups -> scale floor branch
        w[2, :64] = 5e-12                      # tiny maxabs: the two qNg64 floors differ here
    return w


# ---------------------------------------------------------------- IEEE half
def test_f16_decode_exhaustive(oracle):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([oracle.lib.or_f16_to_f32(int(v)) for v in h], np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.all(np.isnan(got[~fin]) == np.isnan(want[~fin]))


def test_f16_encode_rne(oracle):
    rng = np.random.default_rng(7)
    # all halves' exact values, their midpoints (ties) and random floats across the range
    h = np.arange(0, 0x7c00, dtype=np.uint16)
    exact = h.view(np.float16).astype(np.float32)
    mids = ((exact[:-1].astype(np.float64) + exact[1:]) / 2).astype(np.float32)
    rnd = (rng.standard_normal(20000) * np.exp(rng.uniform(-20, 11, 20000))).astype(np.float32)
    vals = np.concatenate([exact, mids, -mids, rnd, np.float32([65504, 65519.99, 65520, 1e-8, 2.0 ** -25, 2.0 ** -24])])
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------- packers vs the reference build
@pytest.mark.parametrize("shape", [(7, 64), (33, 256), (16, 1536)])
def test_q4g64_packer_matches_reference(oracle, ref, shape):
    w = _weights(11, *shape)
    p, s = oracle.quantize_q4g64(w)
    rp = np.zeros_like(p); rs = np.zeros_like(s)
    ref.gguf_quantize_q4g64_error_feedback(_ptr(w), shape[0], shape[1], _ptr(rp), _ptr(rs))
    assert np.array_equal(p, rp) and np.array_equal(s.view(np.uint32), rs.view(np.uint32))


@pytest.mark.parametrize("shape", [(7, 64), (33, 256), (16, 1536)])
def test_q8g64_packer_matches_reference(oracle, ref, shape):
    w = _weights(12, *shape)
    c, s = oracle.quantize_q8g64(w)
    rc = np.zeros_like(c); rs = np.zeros_like(s)
    ref.gguf_quantize_q8g64(_ptr(w), shape[0], shape[1], _ptr(rc), _ptr(rs))
    assert np.array_equal(c, rc) and np.array_equal(s.view(np.uint32), rs.view(np.uint32))


@pytest.mark.parametrize("n", [2, 3, 4, 5, 7, 8, 12, 15])
def test_qng64_gguf_packer_matches_reference(oracle, ref, n):
    w = _weights(13 + n, 9, 192)
    p, s = oracle.quantize_qng64_gguf(w, n)
    rp = np.zeros_like(p); rs = np.zeros_like(s)
    ref.gguf_quantize_qNg64(_ptr(w), 9, 192, n, _ptr(rp), _ptr(rs))
    assert np.array_equal(p, rp) and np.array_equal(s.view(np.uint32), rs.view(np.uint32))


@pytest.mark.parametrize("n", QNG_NS)
def test_qng64_dense_packer_matches_reference(oracle, ref, n):
    w = _weights(31 + n, 9, 192)
    p, s = oracle.quantize_qng64_dense(w, n)
    rp = np.zeros_like(p); rs = np.zeros_like(s)
    assert ref.qng64_quantize_f32(_ptr(w), 9, 192, n, _ptr(rp), _ptr(rs)) == 0
    assert np.array_equal(p, rp) and np.array_equal(s.view(np.uint32), rs.view(np.uint32))


def test_qng64_dense_rejects_n4(oracle, ref):
    w = _weights(3, 4, 64)
    with pytest.raises(ValueError):
        oracle.quantize_qng64_dense(w, 4)
    rp = np.zeros((4, 32), np.uint8); rs = np.zeros((4, 1), np.float32)
    assert ref.qng64_quantize_f32(_ptr(w), 4, 64, 4, _ptr(rp), _ptr(rs)) == -1
    assert ref.qng64_group_bytes(4) == 0 and ref.qng64_group_bytes(5) == 40


def test_qng64_encoders_differ_only_at_the_floor(oracle):
    # gguf_quantize_qNg64 floors scale<1e-12 to 1; qng64_quantize_f32 floors maxabs<=1e-12.
    w = _weights(5, 6, 128)
    pg, sg = oracle.quantize_qng64_gguf(w, 5)
    pd, sd = oracle.quantize_qng64_dense(w, 5)
    assert sg[2, 0] == 1.0 and sd[2, 0] != 1.0          # row 2 group 0: maxabs 1e-13*... differs
    keep = np.ones_like(sg, bool); keep[2, 0] = False
    assert np.array_equal(sg[keep], sd[keep])


def test_q4_0_packer_and_decoder_match_reference(oracle, ref):
    w = _weights(17, 12, 256).ravel()
    b = oracle.quantize_q4_0(w)
    rb = np.zeros_like(b)
    ref.gguf_w_quantize_q4_0(_ptr(w), C.c_int64(w.size), _ptr(rb))
    assert np.array_equal(b, rb)
    d = oracle.decode_q4_0(b, w.size)
    rd = np.zeros_like(d)
    ref.gguf_dequant_row(2, _ptr(b), _ptr(rd), C.c_int64(w.size))        # GGML_TYPE_Q4_0 = 2
    assert np.array_equal(d.view(np.uint32), rd.view(np.uint32))


def test_q4g32h_is_a_lossless_repair_of_q4_0(oracle, ref):
    out, inn = 10, 320
    w = _weights(19, out, inn)
    b = oracle.quantize_q4_0(w.ravel())
    p, s16 = oracle.q4_0_to_q4g32h(b, out, inn)
    d = oracle.decode(5, p, s16, out, inn)
    rd = np.zeros(out * inn, np.float32)
    ref.gguf_dequant_row(2, _ptr(b), _ptr(rd), C.c_int64(out * inn))
    assert np.array_equal(d.ravel().view(np.uint32), rd.view(np.uint32))
    # the nibble convention is q4gemv's: byte b low = column 2b, high = column 2b+1
    q4 = oracle.quantize_q4g32h(w)
    assert np.array_equal(q4[0], p) and np.array_equal(q4[1], s16)


def test_qng64_decode_and_matvec_match_reference(oracle, ref):
    for n in (2, 5, 9, 15):
        w = _weights(23 + n, 8, 256)
        p, s = oracle.quantize_qng64_dense(w, n)
        d = oracle.decode(4, p, s, 8, 256, bits=n)
        for r in range(8):
            for c in range(0, 256, 7):
                grp = p[r, (c // 64) * n * 8:]
                code = ref.qng64_decode_code(grp.ctypes.data_as(C.c_void_p), n, c % 64)
                assert np.float32(code) * s[r, c // 64] == d[r, c]
        x = seeded_normal(99, (3, 256))
        bias = seeded_normal(98, (8,))
        y = oracle.gemm_f32(4, p, s, x, bias=bias, bits=n)
        ry = np.zeros_like(y)
        ref.qng64_matmul_f32(_ptr(p), _ptr(s), n, _ptr(x), _ptr(bias), _ptr(ry), 8, 256, 3)
        assert np.array_equal(y.view(np.uint32), ry.view(np.uint32))


# ---------------------------------------------------------------- the reference's own known answers
def test_qng64_kat(oracle, ref):
    """tools/qng64_dense_test.c:12-36: n=5, 3x64; group_bytes == 40; matvec within 1e-5 of a
    double re-decode."""
    src, x = kat_qng64()
    p, s = oracle.quantize_qng64_dense(src, 5)
    assert p.shape[1] == 40
    y = oracle.gemm_f32(4, p, s, x, bits=5)
    for r in range(3):
        refsum = sum(np.float64(np.float32(oracle.lib.or_qng64_decode_code(p[r].ctypes.data_as(C.c_void_p), 5, q)) * s[r, 0]) * x[q]
                     for q in range(64))
        assert abs(y[r] - np.float32(refsum)) <= 1e-5
    rp = np.zeros_like(p); rs = np.zeros_like(s)
    ref.qng64_quantize_f32(_ptr(src), 3, 64, 5, _ptr(rp), _ptr(rs))
    assert np.array_equal(p, rp)


def _rel_l2_decode(d, ref_w):
    return float(np.sqrt(np.sum((d.astype(np.float64) - ref_w) ** 2) / np.sum(ref_w.astype(np.float64) ** 2)))


def _rel_l2_matvec(oracle, kind, bits, packed, scales, ref_w):
    x = reg_probe()
    ex = expert_struct(kind, bits, packed, scales)
    y = np.array([oracle.lib.or_moe_row(C.byref(ex), 128, C.c_long(r), _ptr(x)) for r in range(16)])
    yref = ref_w.astype(np.float64) @ x.astype(np.float64)
    return float(np.sqrt(np.sum((y - yref) ** 2) / np.sum(yref ** 2)))


def test_regression_control_constants(oracle):
    """tests/regression/test_f2_qng64_n8.c:83-106, test_n2_role_bits_qng64.c:72,134-139 and
    test_f1_mixed_ebits.c:118-132 pin the packers end to end on the mk_tiny_st fixture as
    rel-L2 of decode / matvec against fp32, to 5 decimals."""
    fx = tiny_st()
    e0, e1, dw = fx["L0.e0.w"], fx["L0.e1.w"], fx["dense.w"]
    tol = 2e-5

    def q4(w):
        p, s = oracle.quantize_q4g64(w); return p, s, oracle.decode(1, p, s, 16, 128)

    def q8(w):
        c, s = oracle.quantize_q8g64(w); return c, s, oracle.decode(2, c, s, 16, 128)

    def qn(w, n):
        p, s = oracle.quantize_qng64_gguf(w, n); return p, s, oracle.decode(4, p, s, 16, 128, bits=n)

    checks = []
    p, s, d = q4(e0); checks += [(_rel_l2_decode(d, e0), 0.27455), (_rel_l2_matvec(oracle, 1, 4, p, s, e0), 0.16776)]
    p, s, d = q4(dw); checks += [(_rel_l2_decode(d, dw), 0.29269), (_rel_l2_matvec(oracle, 1, 4, p, s, dw), 0.23906)]
    for w, dec, mv in ((e0, 0.01042, 0.01097), (e1, 0.01121, 0.00924), (dw, 0.01117, 0.01469)):
        c, s, d = q8(w); checks += [(_rel_l2_decode(d, w), dec), (_rel_l2_matvec(oracle, 2, 8, c, s, w), mv)]
    for n, want in zip([2, 3, 5, 6, 7], [1.20871, 0.62646, 0.13574, 0.06342, 0.03119]):
        checks.append((_rel_l2_decode(qn(dw, n)[2], dw), want))
    for n, w, dec, mv in ((7, e0, 0.03007, 0.02358), (7, e1, 0.03396, 0.04540),
                          (9, e0, 0.00775, 0.00459), (9, e1, 0.00807, 0.00718)):
        p, s, d = qn(w, n); checks += [(_rel_l2_decode(d, w), dec), (_rel_l2_matvec(oracle, 4, n, p, s, w), mv)]
    p, s, d = qn(dw, 7); checks.append((_rel_l2_matvec(oracle, 4, 7, p, s, dw), 0.03868))
    p, s, d = qn(dw, 9); checks += [(_rel_l2_decode(d, dw), 0.00766), (_rel_l2_matvec(oracle, 4, 9, p, s, dw), 0.00611)]
    for got, want in checks:
        assert abs(got - want) < tol, (got, want)


def test_n8_matches_independent_plane_redecode(oracle):
    """test_f2_qng64_n8.c:33-68: decode equals an independent bit-plane re-read exactly."""
    fx = tiny_st()
    for name in ("L0.e0.w", "dense.w"):
        w = fx[name]
        p, s = oracle.quantize_qng64_gguf(w, 8)
        d = oracle.decode(4, p, s, 16, 128, bits=8)
        g = p.reshape(16, 2, 8, 8)                      # [row][group][plane][byte]
        bits = np.unpackbits(g, axis=-1, bitorder="little")   # [row][group][plane][64 elems]
        u = np.tensordot(bits.astype(np.int64), 1 << np.arange(8), axes=([2], [0]))   # [row][group][64]
        want = (u - 128).astype(np.float32) * s[:, :, None]
        assert np.array_equal(d.reshape(16, 2, 64), want)
        assert _rel_l2_decode(d, w) < 0.02


def test_n4_qng64_equals_q4g64_values(oracle):
    """gguf_transcode.h:217-223: qNg64 n=4 is value-identical to q4g64 (same codes, same scales)."""
    w = _weights(41, 12, 256)
    p4, s4 = oracle.quantize_q4g64(w)
    pn, sn = oracle.quantize_qng64_gguf(w, 4)
    assert np.array_equal(s4, sn)
    assert np.array_equal(oracle.decode(1, p4, s4, 12, 256), oracle.decode(4, pn, sn, 12, 256, bits=4))


def test_gate9_fixture_and_gather_oracle(oracle, ref):
    """qwen_infer.c:10811-10875 (GATE9): E=4, 6 explicit pairs, n=7; every (pair,row) of the
    gathered product equals an independent double re-decode."""
    g = gate9()
    for e in range(g["E"]):
        p, s = oracle.quantize_qng64_gguf(g["w"][e], 7)
        rp = np.zeros_like(p); rs = np.zeros_like(s)
        ref.gguf_quantize_qNg64(_ptr(np.ascontiguousarray(g["w"][e])), 8, 128, 7, _ptr(rp), _ptr(rs))
        assert np.array_equal(p, rp) and np.array_equal(s, rs)
        for z in np.nonzero(g["idx"] == e)[0]:
            ex = expert_struct(4, 7, p, s)
            xz = np.ascontiguousarray(g["x"][z])
            y = np.array([oracle.lib.or_moe_row(C.byref(ex), 128, C.c_long(r), _ptr(xz)) for r in range(8)])
            d = oracle.decode(4, p, s, 8, 128, bits=7).astype(np.float64)
            assert np.max(np.abs(y - d @ xz.astype(np.float64))) < 1e-12


# ---------------------------------------------------------------- W4A8 / W8A8 semantics
def test_quant_act_rounding_and_floor(oracle):
    # q4gemv.h:188-211: round half AWAY from zero after x*(1/sc), saturating; 1e-8 floor.
    x = np.zeros(64, np.float32)
    x[0] = 127.0                            # sc = 1, inv = 1
    x[1], x[2], x[3], x[4] = 2.5, -2.5, 0.5, -0.5
    x[5], x[6] = -127.0, 126.5
    xq, a = oracle.quant_act_i8(x, 64)
    assert a[0] == np.float32(1.0)
    assert list(xq[:7]) == [127, 3, -3, 1, -1, -127, 127]      # RNE would give 2, -2, 0, 0
    z = np.zeros(256, np.float32)
    zq, za = oracle.quant_act_i8(z, 256)
    assert za[0] == np.float32(np.float32(1e-8) / np.float32(127.0)) and not zq.any()
    # the reverted 'inv = 127/mx' variant differs from 1/(mx/127) on some inputs: prove the
    # oracle follows the reference's two-step reciprocal.
    r = seeded_normal(5, (4096,))
    xq, a = oracle.quant_act_i8(r, 64)
    g = r.reshape(-1, 64)
    mx = np.maximum(np.float32(1e-8), np.abs(g).max(axis=1))
    inv_two = np.float32(1.0) / (mx / np.float32(127.0))
    inv_one = np.float32(127.0) / mx
    assert np.any(inv_two != inv_one)
    assert np.array_equal(a, mx / np.float32(127.0))


@pytest.mark.parametrize("gs", [64, 256])
def test_quant_act_nonfinite_groups(oracle, gs):
    """q4gemv.h:182-206 / q4gemv_g256.h:76-96 on NaN and +-Inf, by the AArch64 instruction
    definitions: FMAX (vmaxq_f32, vmaxvq_f32) returns NaN when an operand is NaN, FCVTZS
    (vcvtq_s32_f32) maps NaN to 0.  A NaN group: mx = NaN, sc = NaN, every code 0.  A +-Inf group:
    mx = +Inf, sc = +Inf, inv = 0, x*inv = +-0 (NaN at the Inf): every code 0.  Groups without a
    non-finite value are untouched, and the fold's 0 * NaN / 0 * Inf makes every output row NaN."""
    x = seeded_normal(17, (4 * gs,))
    clean_q, clean_a = oracle.quant_act_i8(x, gs)
    x[1] = np.nan                                        # group 0: one NaN
    x[gs + 5] = np.inf                                   # group 1: +Inf
    x[2 * gs + 7] = -np.inf                              # group 2: -Inf and a NaN
    x[2 * gs + 9] = np.nan
    xq, a = oracle.quant_act_i8(x, gs)
    assert np.isnan(a[0]) and not xq[:gs].any()
    assert a[1] == np.float32(np.inf) and not xq[gs:2 * gs].any()
    assert np.isnan(a[2]) and not xq[2 * gs:3 * gs].any()
    assert a[3] == clean_a[3] and np.array_equal(xq[3 * gs:], clean_q[3 * gs:])
    # -Inf alone: FMAX over |x| gives +Inf, the same as +Inf
    y = seeded_normal(18, (gs,)); y[3] = -np.inf
    yq, ya = oracle.quant_act_i8(y, gs)
    assert ya[0] == np.float32(np.inf) and not yq.any()
    # the largest finite values quantize normally: the max maps to +-127
    big = seeded_normal(19, (gs,)); big[0] = np.float32(3.0e38); big[1] = np.float32(-3.0e38)
    bq, ba = oracle.quant_act_i8(big, gs)
    assert np.isfinite(ba[0]) and bq[0] == 127 and bq[1] == -127
    # through the fold: every output row of a column with a non-finite group is NaN, the other
    # column is finite
    out, inn = 16, 4 * gs
    w = _weights(91, out, inn)
    kind = 3 if gs == 256 else 1
    if kind == 1:
        p, s = oracle.quantize_q4g64(w); sub = None
    else:
        p, s, sub = oracle.quantize_g256sf(w)
    xm = np.stack([x, seeded_normal(20, (inn,))]).astype(np.float32)
    ym = oracle.matmul_sdot(kind, p, s, xm, sub=sub)
    assert np.isnan(ym[0]).all() and np.isfinite(ym[1]).all()


@pytest.mark.parametrize("kind", [1, 2, 3])
def test_sdot_gemm_equals_dequantized_product(oracle, kind):
    """Identity: the W4A8/W8A8 result equals the fp32 product of the decoded weights with the
    de-quantized activation (xq * ascale), up to fp32 rounding; batched == per column."""
    out, inn, M = 24, 1024, 5
    w = _weights(50 + kind, out, inn)
    x = seeded_normal(60 + kind, (M, inn))
    bias = seeded_normal(70, (out,))
    if kind == 1:
        p, s = oracle.quantize_q4g64(w); sub = None; gs = 64
    elif kind == 2:
        p, s = oracle.quantize_q8g64(w); sub = None; gs = 64
    else:
        p, s, sub = oracle.quantize_g256sf(w); gs = 256
    y = oracle.matmul_sdot(kind, p, s, x, bias=bias, sub=sub)
    xq, a = oracle.quant_act_i8(x, gs)
    xd = (xq.astype(np.float64).reshape(M, -1, gs) * a[:, :, None]).reshape(M, inn)
    wd = oracle.decode(kind, p, s, out, inn, sub=sub).astype(np.float64)
    want = xd @ wd.T + bias
    assert np.max(np.abs(y - want)) / np.max(np.abs(want)) < 2e-6
    for m in range(M):
        ym = oracle.matmul_sdot(kind, p, s, x[m], bias=bias, sub=sub)
        assert np.array_equal(ym, y[m])


def test_fp32_gemv_equals_double_product(oracle):
    out, inn = 20, 512
    w = _weights(81, out, inn)
    x = seeded_normal(82, (3, inn))
    for kind in (1, 2, 5):
        if kind == 1:
            p, s = oracle.quantize_q4g64(w)
        elif kind == 2:
            p, s = oracle.quantize_q8g64(w)
        else:
            p, s = oracle.quantize_q4g32h(w)
        y = oracle.gemm_f32(kind, p, s, x)
        wd = oracle.decode(kind, p, s, out, inn).astype(np.float64)
        assert np.array_equal(y, (x.astype(np.float64) @ wd.T).astype(np.float32))


def test_g256sf_packer_roundtrip(oracle):
    """Build-defined packer: sub codes in [1,63], effective scale wsuper*sub/63 >= s64 so no
    code saturates beyond the EF clamp; decode rel-L2 comparable to q4g64."""
    w = _weights(90, 32, 1536, outliers=False, zero_rows=False)
    p, ws, sub = oracle.quantize_g256sf(w)
    assert sub.min() >= 1 and sub.max() <= 63
    d = oracle.decode(3, p, ws, 32, 1536, sub=sub)
    p4, s4 = oracle.quantize_q4g64(w)
    d4 = oracle.decode(1, p4, s4, 32, 1536)
    assert _rel_l2_decode(d, w) < 1.2 * _rel_l2_decode(d4, w)


def _equal_subgroup_max(w):
    """Every 64-subgroup of each 256-group gets the same max |w|: the subgroup's largest element is
    set (sign kept) to the largest magnitude of its 256-group."""
    w = w.copy()
    out, inn = w.shape
    g = w.reshape(out, inn // 256, 4, 64)
    a = np.abs(g)
    big = a.max(axis=(2, 3))                                   # [out][n256]
    idx = a.argmax(axis=3)                                     # [out][n256][4]
    o, s, k = np.meshgrid(np.arange(out), np.arange(inn // 256), np.arange(4), indexing="ij")
    sign = np.where(g[o, s, k, idx] < 0, -1.0, 1.0).astype(np.float32)
    g[o, s, k, idx] = sign * big[:, :, None]
    return g.reshape(out, inn)


@pytest.mark.parametrize("shape", [(5, 256), (24, 1536), (9, 8960)])
def test_g256sf_packer_reduces_to_reference_q4g64(oracle, ref, shape):
    """Where the four 64-subgroups of every 256-group share their max |w|, the g256sf packer must
    be the reference's q4g64 error-feedback packer (gguf_transcode.c:24-68, built from the
    reference's own C in oracle/_ref): sub = 63 everywhere, the codes byte for byte and wsuper
    equal to its per-64 scales bit for bit.  A dropped error-feedback step, a wrong rounding or
    nibble order, or a sub-code off by one fails here."""
    w = _equal_subgroup_max(_weights(95, *shape, outliers=True, zero_rows=False))
    p, ws, sub = oracle.quantize_g256sf(w)
    rp = np.zeros_like(p)
    rs = np.zeros((shape[0], shape[1] // 64), np.float32)
    ref.gguf_quantize_q4g64_error_feedback(_ptr(w), shape[0], shape[1], _ptr(rp), _ptr(rs))
    assert np.all(sub == 63)
    assert np.array_equal(p, rp)
    rs4 = rs.reshape(shape[0], -1, 4)
    assert np.all(rs4 == rs4[:, :, :1])                       # the reference's four scales agree
    assert np.array_equal(ws.view(np.uint32), np.ascontiguousarray(rs4[:, :, 0]).view(np.uint32))


def test_g256sf_sub_code_is_minimal(oracle):
    """sub is the smallest integer in [1, 63] whose effective scale wsuper * sub / 63 covers the
    subgroup's max |w| / 7 (up to one fp32 rounding), and wsuper is the largest subgroup scale."""
    w = _weights(96, 40, 2048, outliers=True, zero_rows=False)
    w[3, :256] *= np.float32(1e-3)                             # a 256-group of tiny subgroups
    w[4, 64:128] = 0.0                                         # one all-zero subgroup
    p, ws, sub = oracle.quantize_g256sf(w)
    s64 = (np.abs(w).reshape(40, -1, 64).max(axis=2) / np.float32(7.0)).astype(np.float32).astype(np.float64)
    wsb = np.repeat(ws.astype(np.float64), 4, axis=1)
    assert np.array_equal(ws.astype(np.float64), s64.reshape(40, -1, 4).max(axis=2))
    eff = wsb * sub / 63.0
    assert np.all(eff >= s64 * (1 - 2.0 ** -22))
    lower = wsb * (sub.astype(np.float64) - 1) / 63.0
    assert np.all((sub == 1) | (lower < s64 * (1 + 2.0 ** -22)))
    assert sub.min() >= 1 and sub.max() <= 63


# ---------------------------------------------------------------- MoE
def test_mixed_qng64_decode_uniform_equals_dense(oracle):
    """A mixed tensor whose cells all have the same n is the qng64_dense layout (qng64_dense.c:19-27
    vs mlx_moe.cpp:1708-1722): or_decode_qng64_mixed equals or_decode_qng64 on the same bytes."""
    from oracle_ffi import mixed_qng64_py_decode
    out, inn = 9, 256
    for n in (2, 3, 4, 5, 7, 8, 12, 15):
        w = seeded_normal(300 + n, (out, inn), 0.02)
        planes, scales = oracle.quantize_qng64_gguf(w, n)
        cells = out * inn // 64
        offsets = (np.arange(cells + 1, dtype=np.uint32) * np.uint32(n * 8)).astype(np.uint32)
        bits = np.full(cells, n, np.uint8)
        got = oracle.decode_qng64_mixed(planes.reshape(-1), offsets, bits, scales.reshape(-1), out, inn)
        ref = oracle.decode(4, planes, scales, out, inn, bits=n)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), n
        py = mixed_qng64_py_decode(planes.reshape(-1), offsets, bits, scales.reshape(-1), out, inn)
        assert np.array_equal(py.view(np.uint32), ref.view(np.uint32)), n


def test_mixed_qng64_decode_random_widths(oracle):
    """Per-cell widths 2..15 (4 included, which the dense packer refuses) against the independent
    Python bit-plane decode, bit for bit; the extreme codes of every width are reached."""
    from oracle_ffi import mixed_qng64_py_decode, mixed_qng64_random
    rng = np.random.default_rng(31)
    out, inn = 7, 320
    planes, offsets, bits, scales = mixed_qng64_random(rng, out, inn, list(range(2, 16)))
    planes[:int(offsets[1])] = 0xFF                  # cell 0: all-ones code, 2^(n-1) - 1
    planes[int(offsets[1]):int(offsets[2])] = 0      # cell 1: all-zero code, -2^(n-1)
    got = oracle.decode_qng64_mixed(planes, offsets, bits, scales, out, inn)
    ref = mixed_qng64_py_decode(planes, offsets, bits, scales, out, inn)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    n0, n1 = int(bits[0]), int(bits[1])
    assert np.all(got[0, :64] == np.float32((1 << (n0 - 1)) - 1) * scales[0])
    assert np.all(got[0, 64:128] == np.float32(-(1 << (n1 - 1))) * scales[1])


def test_router_logits_match_sequential_double(oracle):
    """or_moe_router_logits (moe_matvec_f32, qwen_infer.c:3460-3466, + bias) against a pure-Python
    loop in the reference order: Python floats are IEEE doubles and a product of two floats is
    exact in double, so `acc += w * x` rounds exactly as the C loop does.  Bit for bit."""
    rng = np.random.default_rng(77)
    T, E, H = 3, 8, 96
    w = (rng.standard_normal((E, H)) * 0.05).astype(np.float32)
    x = rng.standard_normal((T, H)).astype(np.float32)
    x[1, ::7] *= np.float32(1e4)                       # wide dynamic range: the double sum rounds
    b = (rng.standard_normal(E) * 0.1).astype(np.float32)
    got = oracle.router_logits(w, x, b)
    got_nb = oracle.router_logits(w, x)
    for t in range(T):
        for e in range(E):
            acc = 0.0
            for c in range(H):
                acc += float(w[e, c]) * float(x[t, c])
            ref = np.float32(acc)
            assert got_nb[t, e].view(np.uint32) == ref.view(np.uint32)
            assert got[t, e].view(np.uint32) == np.float32(ref + b[e]).view(np.uint32)
    # a float accumulator (the plausible mistake) differs on the wide-range row
    accf = np.float32(0.0)
    for c in range(H):
        accf = np.float32(accf + w[0, c] * x[1, c])
    assert accf != got_nb[1, 0]


def test_route_matches_brute_force(oracle):
    lg = seeded_normal(100, (64, 64))
    idx, wts = oracle.route(lg, 6)
    for t in range(64):
        e = np.exp(lg[t].astype(np.float64) - lg[t].max())
        prob = e / e.sum()
        order = np.argsort(-prob, kind="stable")[:6]
        assert list(order) == list(idx[t])
        assert np.allclose(wts[t], prob[order], rtol=1e-6)
    idx2, w2 = oracle.route(lg, 6, renorm=True)
    assert np.array_equal(idx, idx2) and np.allclose(w2.sum(axis=1), 1.0, atol=1e-6)


def _small_moe(oracle, seed, E=8, H=128, I=64, Ish=128, kinds=(5, 2, 4)):
    rng = np.random.default_rng(seed)
    keep = []

    def mk(kind, bits, out, inn, s):
        w = seeded_normal(s, (out, inn), 0.02)
        if kind == 5:
            p, sc = oracle.quantize_q4g32h(w)
        elif kind == 2:
            p, sc = oracle.quantize_q8g64(w)
        else:
            p, sc = oracle.quantize_qng64_dense(w, bits)
        keep.append((p, sc))
        return expert_struct(kind, bits, p, sc)

    gate, up, down = [], [], []
    for e in range(E):
        kind = kinds[rng.integers(len(kinds))]
        bits = int(rng.integers(7, 16)) if kind == 4 else (8 if kind == 2 else 4)
        gate.append(mk(kind, bits, I, H, seed * 100 + e * 3))
        up.append(mk(kind, bits, I, H, seed * 100 + e * 3 + 1))
        down.append(mk(kind, bits, H, I, seed * 100 + e * 3 + 2))
    sh = [mk(2, 8, Ish, H, seed + 7), mk(2, 8, Ish, H, seed + 8), mk(2, 8, H, Ish, seed + 9)]
    arr = lambda lst: (type(lst[0]) * len(lst))(*lst)
    return dict(gate=arr(gate), up=arr(up), down=arr(down), sh=sh, keep=keep, E=E, H=H, I=I, Ish=Ish)


def test_moe_bucketed_equals_naive(oracle):
    """moe_ffn_batched (bucketed) vs moe_ffn_naive_batched: the gather invariance; only the fp32
    order of the weighted sum differs."""
    m = _small_moe(oracle, 3)
    T, K = 8, 3
    x = seeded_normal(5, (T, m["H"]))
    idx, wts = oracle.route(seeded_normal(6, (T, m["E"])), K)
    outs = []
    for fn in (oracle.lib.or_moe_ffn_bucketed, oracle.lib.or_moe_ffn_naive):
        o = np.zeros((T, m["H"]), np.float32)
        fn(m["gate"], m["up"], m["down"], m["E"], C.byref(m["sh"][0]), C.byref(m["sh"][1]), C.byref(m["sh"][2]),
           m["H"], m["I"], m["Ish"], T, K, _ptr(x), _ptr(idx), _ptr(wts), _ptr(o))
        outs.append(o)
    assert np.max(np.abs(outs[0] - outs[1])) <= 1e-5 * np.max(np.abs(outs[1]))
    assert np.abs(outs[0]).max() > 0


def test_moe_row_equals_decoded_double_dot(oracle):
    w = seeded_normal(9, (16, 256), 0.02)
    x = seeded_normal(10, (256,))
    for kind, bits in ((5, 4), (2, 8), (4, 7), (4, 15), (1, 4)):
        if kind == 5:
            p, s = oracle.quantize_q4g32h(w)
        elif kind == 2:
            p, s = oracle.quantize_q8g64(w)
        elif kind == 1:
            p, s = oracle.quantize_q4g64(w)
        else:
            p, s = oracle.quantize_qng64_dense(w, bits)
        ex = expert_struct(kind, bits, p, s)
        y = np.array([oracle.lib.or_moe_row(C.byref(ex), 256, C.c_long(r), _ptr(x)) for r in range(16)])
        d = oracle.decode(kind, p, s, 16, 256, bits=bits).astype(np.float64)
        assert np.allclose(y, d @ x.astype(np.float64), rtol=0, atol=1e-12)


def test_moe_ffn_equals_decoded_pipeline(oracle):
    """The FFN oracle (through the tests' moe_ffn helper) against a dense float64 pipeline over
    weights decoded by or_decode: pins the plumbing (token rows, expert ids, routing weights,
    shared expert added once per token) independently of or_moe_row's per-format decode."""
    from oracle_ffi import moe_ffn
    E, H, I, Ish, K, T = 6, 128, 64, 128, 2, 5
    fm = [(5, 0), (2, 0), (4, 9)]

    def mk(e, out, inn, s):
        k, b = fm[e % 3]
        w = seeded_normal(s, (out, inn), 0.02)
        if k == 5:
            p, sc = oracle.quantize_q4g32h(w)
        elif k == 2:
            p, sc = oracle.quantize_q8g64(w)
        else:
            p, sc = oracle.quantize_qng64_dense(w, b)
        return (k, b if k == 4 else (8 if k == 2 else 4), p, sc)

    gate = [mk(e, I, H, 300 + 3 * e) for e in range(E)]
    up = [mk(e, I, H, 301 + 3 * e) for e in range(E)]
    down = [mk(e, H, I, 302 + 3 * e) for e in range(E)]
    shared = (mk(1, Ish, H, 400), mk(1, Ish, H, 401), mk(1, H, Ish, 402))
    x = seeded_normal(403, (T, H))
    idx, w = oracle.route(seeded_normal(404, (T, E)), K, True)
    got = moe_ffn(oracle, gate, up, down, shared, H, I, x, idx, w)

    def dec(d, out, inn):
        return oracle.decode(d[0], d[2], d[3], out, inn, bits=d[1]).astype(np.float64)

    def mlp(g, u, dn, inter, xt):
        a = dec(g, inter, H) @ xt
        b = dec(u, inter, H) @ xt
        return dec(dn, H, inter) @ (a / (1.0 + np.exp(-a)) * b)

    want = np.zeros((T, H))
    for t in range(T):
        xt = x[t].astype(np.float64)
        for k in range(K):
            e = idx[t, k]
            want[t] += float(w[t, k]) * mlp(gate[e], up[e], down[e], I, xt)
        want[t] += mlp(*shared, Ish, xt)
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))
    # dropping the shared expert or one routed pair moves the result far outside that bar
    no_sh = moe_ffn(oracle, gate, up, down, None, H, I, x, idx, w)
    assert np.max(np.abs(no_sh - want)) > 1e-3 * np.max(np.abs(want))


def _af_descs(oracle, out=24, inn=256, seed=11):
    """One descriptor per MoE row kind: (kind, bits, packed, scales[, bias])."""
    rng = np.random.default_rng(seed)
    w = seeded_normal(seed, (out, inn), 0.02)
    ng = inn // 64
    p1, s1 = oracle.quantize_q4g64(w)
    p2, s2 = oracle.quantize_q8g64(w)
    p4, s4 = oracle.quantize_qng64_dense(w, 9)
    p5, s5 = oracle.quantize_q4g32h(w)
    nib = rng.integers(0, 256, (out, inn // 2), dtype=np.uint8)
    sa = (rng.random((out, ng), dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    ba = (rng.standard_normal((out, ng), dtype=np.float32) * np.float32(0.03)).astype(np.float32)
    f16 = w.astype(np.float16).view(np.uint16)
    return {1: (1, 4, p1, s1), 2: (2, 8, p2, s2), 4: (4, 9, p4, s4), 5: (5, 4, p5, s5),
            6: (6, 4, nib, sa, ba), 7: (7, 16, f16, None), 8: (8, 32, w, None)}


def test_moe_decode_and_row_agree_for_every_kind(oracle):
    """or_moe_row (the per-kind row loops of moe_matvec_af_row) equals the double dot over
    or_moe_decode (moe_decode_af) -- two separate restatements of each kind's decode."""
    from oracle_ffi import expert_array, moe_decode
    out, inn = 24, 256
    x = seeded_normal(12, (inn,))
    for kind, d in _af_descs(oracle, out, inn).items():
        arr, keep = expert_array([d])
        for r in (0, 7, out - 1):
            dec = moe_decode(oracle, d, out, inn, r, range(inn)).astype(np.float64)
            row = oracle.lib.or_moe_row(arr, inn, C.c_long(r), _ptr(x))
            assert abs(row - dec @ x.astype(np.float64)) <= 1e-12 * max(1.0, abs(row)), kind


def test_moe_decode_dense_and_affine_fixed_points(oracle):
    """fp16 decode == numpy's float16 widening; fp32 decode returns the stored float; int4 affine
    with bias = -8*scale reproduces the symmetric int4 decode to within one rounding."""
    from oracle_ffi import moe_decode
    out, inn = 24, 256
    d = _af_descs(oracle, out, inn)
    f16 = d[7][2]
    for r in (0, 5):
        got = moe_decode(oracle, d[7], out, inn, r, range(inn))
        assert np.array_equal(got, f16[r].view(np.float16).astype(np.float32))
        assert np.array_equal(moe_decode(oracle, d[8], out, inn, r, range(inn)), d[8][2][r])
    p1, s1 = d[1][2], d[1][3]
    aff = (6, 4, p1, s1, (np.float32(-8.0) * s1).astype(np.float32))
    for r in (0, 3, 11):
        sym = moe_decode(oracle, d[1], out, inn, r, range(inn))
        af = moe_decode(oracle, aff, out, inn, r, range(inn))
        tol = np.repeat(s1[r], 64) * np.float32(2 ** -20)
        assert np.all(np.abs(af - sym) <= tol)


def test_pool_moe_ffn_equals_bucketed(oracle):
    """The CPU baseline's threaded MoE FFN (rows of every expert matvec over the pool) gives the
    single-threaded bucketed FFN's outputs bit for bit (each row is one thread's sequential sum)."""
    import ctypes as C
    from oracle_ffi import _ptr, expert_array, moe_ffn
    E, H, I, Ish, T, K = 6, 128, 64, 96, 5, 2
    rng = np.random.default_rng(700)
    def d(kind, o, i, s):
        w = seeded_normal(s, (o, i), 0.02)
        p, sc = oracle.quantize_q4g32h(w) if kind == 5 else oracle.quantize_qng64(w, 7)
        return (kind, 4 if kind == 5 else 7, p, sc)
    gate = [d(5 if e % 2 else 4, I, H, 710 + e) for e in range(E)]
    up = [d(5 if e % 2 else 4, I, H, 720 + e) for e in range(E)]
    down = [d(5 if e % 2 else 4, H, I, 730 + e) for e in range(E)]
    shared = (d(5, Ish, H, 740), d(5, Ish, H, 741), d(5, H, Ish, 742))
    x = seeded_normal(750, (T, H))
    idx, w = oracle.route(seeded_normal(751, (T, E)), K)
    ref = moe_ffn(oracle, gate, up, down, shared, H, I, x, idx, w)
    (ga, k1), (ua, k2), (da, k3), (sa, k4) = expert_array(gate), expert_array(up), expert_array(down), expert_array(list(shared))
    out = np.zeros((T, H), np.float32)
    pool = oracle.lib.or_pool_create(3, 1)
    z = C.sizeof(sa[0])
    oracle.lib.or_pool_moe_ffn_bucketed(C.c_void_p(pool), ga, ua, da, E, C.byref(sa, 0), C.byref(sa, z), C.byref(sa, 2 * z),
                                        H, I, Ish, T, K, _ptr(x), _ptr(idx), _ptr(w), _ptr(out))
    oracle.lib.or_pool_destroy(pool)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


def test_swiglu_pins(oracle):
    """or_swiglu (swiglu, qwen_infer.c:726-733): against numpy's float64 exp rounded once to float32,
    then the same float steps (g / (1 + e)) * u; special values; and within 1 ulp of the float-exp
    form the reference evaluates (moe_swiglu_inplace's expf)."""
    rng = np.random.default_rng(77)
    g = np.concatenate([rng.standard_normal(4000).astype(np.float32) * np.float32(4),
                        np.array([0.0, -0.0, 88.0, -88.0, 104.0, -104.0, 1e-30, -1e-30, np.inf, -np.inf, np.nan], np.float32)])
    u = rng.standard_normal(g.size).astype(np.float32)
    u[-11:] = 1.5
    with np.errstate(all="ignore"):
        e = np.exp(-g.astype(np.float64)).astype(np.float32)
        want = (g / (np.float32(1) + e)) * u
    got = oracle.swiglu(g, u)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)) or np.array_equal(got, want, equal_nan=True)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert got[-11] == 0 and got[-9] == np.float32(88.0) * np.float32(1.5)      # silu(0) = 0; silu(88) ~ 88
    assert np.isnan(got[-2]) and np.isnan(got[-1])                              # -inf / inf and NaN propagate
    ref = np.array(g, np.float32)
    gate = ref.copy()
    import ctypes as C
    oracle.lib.or_moe_swiglu_inplace(C.c_void_p(gate.ctypes.data), C.c_void_p(u.ctypes.data), g.size)  # float expf form
    fin = np.isfinite(got) & np.isfinite(gate)
    ulp = np.abs(got[fin].view(np.int32).astype(np.int64) - gate[fin].view(np.int32).astype(np.int64))
    assert ulp.max() <= 2


def test_mxfp4_decode_matches_reference(oracle, ref):
    """The oracle's MXFP4 arms (moe_decode_af / moe_matvec_af_row, qwen_infer.c:2584-2595, :2702-2725)
    against oracle/_ref's gguf_quants.c: every exponent byte 0..255 and every code, element by
    element against gguf_dequant_row(MXFP4 = 39), and the row dot against the decoded row in double
    (pairs j, j+16 summed per the reference's order)."""
    from oracle_ffi import moe_decode, moe_matvec, mxfp4_blocks
    ref.gguf_e8m0_to_fp32_half.restype = C.c_float
    ref.gguf_e8m0_to_fp32_half.argtypes = [C.c_uint8]
    ref.gguf_mxfp4_nibble.restype = C.c_int8
    ref.gguf_mxfp4_nibble.argtypes = [C.c_int]
    oracle.lib.or_mx_scale.restype = C.c_float
    oracle.lib.or_mx_scale.argtypes = [C.c_uint8]
    for b in range(256):
        a, r = np.float32(oracle.lib.or_mx_scale(b)), np.float32(ref.gguf_e8m0_to_fp32_half(b))
        assert a.view(np.uint32) == r.view(np.uint32), b
    assert [oracle.lib.or_mx_value(c) for c in range(16)] == [ref.gguf_mxfp4_nibble(c) for c in range(16)]
    rng = np.random.default_rng(40)
    out, inn = 16, 256
    blk = mxfp4_blocks(rng, out, inn, 0, 256)                 # every exponent byte, subnormal scales included
    blk[0, :, 0] = np.arange(inn // 32, dtype=np.uint8)      # 0 and 1 (the subnormal patterns) for sure
    blk[1, :, 0] = 255 - np.arange(inn // 32, dtype=np.uint8)
    rd = np.zeros(out * inn, np.float32)
    ref.gguf_dequant_row(39, _ptr(blk), _ptr(rd), C.c_int64(out * inn))       # GGML_TYPE_MXFP4 = 39
    rd = rd.reshape(out, inn)
    desc = (9, 4, blk, None)
    for r in (0, 1, 7, 15):
        got = moe_decode(oracle, desc, out, inn, r, range(inn))
        assert np.array_equal(got.view(np.uint32), rd[r].view(np.uint32)), r
    blk = mxfp4_blocks(rng, out, inn)
    desc = (9, 4, blk, None)
    rd = np.zeros(out * inn, np.float32)
    ref.gguf_dequant_row(39, _ptr(blk), _ptr(rd), C.c_int64(out * inn))
    rd = rd.reshape(out, inn)
    x = rng.standard_normal(inn).astype(np.float32)
    want = np.zeros(out, np.float64)
    for r in range(out):
        acc = 0.0
        for b in range(inn // 32):
            for j in range(16):
                c0 = 32 * b
                acc += float(rd[r, c0 + j]) * float(x[c0 + j]) + float(rd[r, c0 + j + 16]) * float(x[c0 + j + 16])
        want[r] = acc
    assert np.array_equal(moe_matvec(oracle, desc, out, inn, x), want.astype(np.float32))


def test_g256plain_row_pins(oracle):
    """or_gemm_g256plain_sdot (q4gemv_g256.h:102-130) at power-of-two weight and activation scales,
    where every term (float)isum * ws * as is exact: the output then equals a float32 running sum,
    in group order, of exact integer sums computed here from the nibbles (low = even column) and
    the oracle's own int8 activation codes -- which pins the nibble order, the 256-groups and the
    pairing of weight and activation groups; a dropped -8 or a group off by one fails it."""
    rng = np.random.default_rng(33)
    out, inn, M = 12, 1024, 3
    pk = rng.integers(0, 256, (out, inn // 2), dtype=np.uint8)
    ws = np.ldexp(np.float32(1), rng.integers(-12, -4, (out, inn // 256))).astype(np.float32)
    x = rng.standard_normal((M, inn)).astype(np.float32)
    xq, asc = oracle.quant_act_i8(x, 256)
    asc = np.ldexp(np.float32(1), np.round(np.log2(asc)).astype(np.int32)).astype(np.float32)   # power-of-two
    nib = np.empty((out, inn), np.int64)
    nib[:, 0::2] = pk & 15
    nib[:, 1::2] = pk >> 4
    y = np.zeros((M, out), np.float32)
    oracle.lib.or_gemm_g256plain_sdot(C.c_void_p(pk.ctypes.data), C.c_void_p(ws.ctypes.data),
                                       C.c_void_p(np.ascontiguousarray(xq).ctypes.data), C.c_void_p(asc.ctypes.data),
                                       None, C.c_void_p(y.ctypes.data), out, inn, M)
    for m in range(M):
        for r in range(out):
            acc = np.float32(0)
            for g in range(inn // 256):
                s = int(np.sum((nib[r, g * 256:(g + 1) * 256] - 8) * xq[m, g * 256:(g + 1) * 256].astype(np.int64)))
                acc = np.float32(acc + np.float32(s) * ws[r, g] * asc[m, g])
            assert y[m, r] == acc, (m, r)
