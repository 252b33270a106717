"""Property tests of the oracle (hypothesis, CPU): invariants of the reference's quantizers,
GEMM and attention that a dropped term, a flipped sign or a transposed operand in the
restatement would break on some input.  The oracle is test infrastructure; these tests pin it
beside the closed forms, torch restatements and golden vectors of the other oracle tests."""
import numpy as np
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st
from hypothesis.extra.numpy import arrays

from oracle import attention as oa
from oracle import linear as ol
from oracle.numerics import e4m3_decode, e4m3_encode

F32 = np.float32
SETTINGS = settings(max_examples=40, deadline=None, suppress_health_check=[HealthCheck.too_slow])

# row values away from fp32's subnormal range, so that scaling by powers of two is exact
ROW_VALUE = st.one_of(st.just(0.0), st.floats(min_value=2.0 ** -10, max_value=3072.0, width=32),
                      st.floats(min_value=-3072.0, max_value=-(2.0 ** -10), width=32))
ROWS = arrays(F32, st.tuples(st.integers(1, 4), st.integers(1, 96)), elements=ROW_VALUE)


@SETTINGS
@given(ROWS)
def test_quantize_rows_scale_and_error_bound(x):
    """scale = max(max|x|, 1e-12) / 448 (fp32); decode(code) * scale is x rounded to e4m3's
    three mantissa bits: within 2^-4 |x| (normal codes) or 2^-10 scale (subnormal codes)."""
    codes, scale = ol.quantize_rows(x)
    amax = np.max(np.abs(x), axis=1, keepdims=True)
    np.testing.assert_array_equal(scale, (np.fmax(amax, F32(1e-12)) / F32(448.0)).astype(F32))
    deq = e4m3_decode(codes).astype(np.float64) * scale.astype(np.float64)
    err = np.abs(deq - x.astype(np.float64))
    bound = np.maximum(2.0 ** -4 * np.abs(x), 2.0 ** -10 * scale) * (1 + 1e-6)
    assert np.all(err <= bound)
    # the row maximum lands on +-448 exactly
    rows = amax[:, 0] > 0
    assert np.all(np.max(np.abs(e4m3_decode(codes[rows])), axis=1) == 448.0)


@SETTINGS
@given(ROWS, st.integers(-8, 8))
def test_quantize_rows_sign_and_power_of_two_invariance(x, k):
    """Negating a row flips every code's sign bit (zeros included: -0 is code 0x80); scaling a
    row by 2^k leaves the codes unchanged and multiplies the scale by exactly 2^k."""
    codes, scale = ol.quantize_rows(x)
    neg_codes, neg_scale = ol.quantize_rows(-x)
    np.testing.assert_array_equal(neg_codes, codes ^ np.uint8(0x80))
    np.testing.assert_array_equal(neg_scale, scale)
    big_codes, big_scale = ol.quantize_rows((x * F32(2.0 ** k)).astype(F32))
    rows = np.max(np.abs(x), axis=1) > 0
    np.testing.assert_array_equal(big_codes[rows], codes[rows])
    np.testing.assert_array_equal(big_scale[rows], (scale[rows] * F32(2.0 ** k)).astype(F32))


@SETTINGS
@given(arrays(F32, st.integers(2, 200), elements=st.floats(min_value=-460, max_value=460, width=32)))
def test_e4m3_encode_is_monotonic_and_nearest(v):
    """Encoding is monotonic on [-460, 460] and picks a nearest e4m3 value (RNE on ties)."""
    v = np.sort(v)
    d = e4m3_decode(e4m3_encode(np.clip(v, -448, 448)))
    assert np.all(np.diff(d) >= 0)
    grid = np.unique(e4m3_decode(np.arange(256, dtype=np.uint8)[(np.arange(256) & 0x7F) != 0x7F]))
    c = np.clip(v, -448, 448).astype(np.float64)
    nearest = np.min(np.abs(grid[None, :] - c[:, None]), axis=1)
    np.testing.assert_array_equal(np.abs(d - c), nearest)


FINITE_CODES = st.integers(0, 253).map(lambda c: c + (c >= 0x7F))  # every code but the NaNs


@SETTINGS
@given(st.integers(1, 12), st.integers(1, 12), st.integers(1, 48), st.data())
def test_scaled_mm_transpose_and_scale_linearity(M, N, K, data):
    """scaled_mm(x8, w8, sa, sw)^T = scaled_mm(w8, x8, sw, sa) (the operands' roles are
    symmetric), and doubling sa doubles the bias-free output exactly."""
    x8 = np.array(data.draw(st.lists(FINITE_CODES, min_size=M * K, max_size=M * K)), np.uint8).reshape(M, K)
    w8 = np.array(data.draw(st.lists(FINITE_CODES, min_size=N * K, max_size=N * K)), np.uint8).reshape(N, K)
    sa = np.array(data.draw(st.lists(st.floats(2.0 ** -10, 4.0, width=32), min_size=M, max_size=M)), F32)
    sw = np.array(data.draw(st.lists(st.floats(2.0 ** -10, 4.0, width=32), min_size=N, max_size=N)), F32)
    out = ol.scaled_mm(x8, w8, sa, sw)
    np.testing.assert_array_equal(out.T, ol.scaled_mm(w8, x8, sw, sa))
    np.testing.assert_array_equal(ol.scaled_mm(x8, w8, (2 * sa).astype(F32), sw), (2 * out).astype(F32))


@settings(max_examples=15, deadline=None, suppress_health_check=[HealthCheck.too_slow])
@given(st.integers(1, 130), st.integers(1, 300), st.integers(0, 2 ** 31 - 1))
def test_attention_output_is_a_convex_combination_of_v(Sq, Sk, seed):
    """Every P code is >= 0 and the row sum l > 0 (the row maximum's code is 56 on the first
    tile and never flushes later), so each output is a weighted mean of the dequantized V
    values of its channel: inside their range (fp32 rounding aside)."""
    rng = np.random.default_rng(seed)
    B, H, D = 1, 1, 64
    q = rng.standard_normal((B, H, Sq, D)).astype(F32)
    k = rng.standard_normal((B, H, Sk, D)).astype(F32)
    v = (rng.standard_normal((B, H, Sk, D)) * rng.uniform(0.1, 10.0)).astype(F32)
    o, inter = oa.fp8_attention(q, k, v, out_dtype="fp32")
    vdeq = e4m3_decode(inter["v8t"]).astype(np.float64).transpose(0, 1, 3, 2) * inter["sv"][:, :, None, :]
    lo, hi = vdeq.min(axis=2, keepdims=True), vdeq.max(axis=2, keepdims=True)
    slack = 1e-5 * np.abs(vdeq).max()
    assert np.all(o >= lo - slack) and np.all(o <= hi + slack)
