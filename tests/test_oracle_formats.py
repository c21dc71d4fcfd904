"""Pins the oracle's restatement of the block formats beyond Q8_0 / Q4_0 (oracle/formats.c):
FP8 E4M3 / E5M2 (ferrum_gguf/src/codec/fp8.rs), MXFP4 (mxfp4.rs), Q2_K (q2k.rs) and the
read-only GGUF block types (blocks.rs). The known answers restate the reference's own unit tests
(fp8/tests.rs, mxfp4/tests.rs, q2k/tests.rs, blocks/tests.rs); where those leave room, an
independent numpy statement of the format (exhaustive over all codes, or a second decoder
written from the ggml layout) checks the C code.

Q2_K's encoder (ggml's make_qkx2_quants search) has no golden bytes in the reference; besides
the reference's properties (error bounds, zero / constant / negative blocks, determinism and
block independence), its bytes are pinned by a second statement of the search written here in
numpy (vectorised over sub-blocks, f32 throughout, sequential sums by cumsum, the nearest_int
magic by its bit definition, f16 by numpy's IEEE cast), which must give the C oracle's bytes on
data that reaches every branch; the same statement with one search constant perturbed (rmin,
rdelta, the step count, the negative-min clamp, the grid's moving min) must not, which shows the data exercises them.
Because a misreading both statements shared would pass that, the C oracle's search result is also
checked against what the mathematics fixes, with no search restated: each sub-block's (scale,
min) is the first grid or the |x|-weighted least-squares fit of its levels (min clamped at 0), its
weighted deviation is no worse than the first grid's, and the bytes pack the nearest 4-bit codes
and the nearest levels to the decoder's own rounded scales. Planted mistakes (unweighted fit,
worse candidate kept, clamp dropped, min sign flipped, levels not re-fitted) each break them."""
import math

import numpy as np
import pytest


def f16b(v: float) -> list:
    h = int(np.float16(v).view(np.uint16))
    return [h & 0xFF, h >> 8]


# ---- FP8 ----

def fp8_value(e5m2: bool, code: int) -> float:
    """Independent statement of the two OCP formats (sign, exponent, mantissa fields)."""
    eb, mb, bias = (5, 2, 15) if e5m2 else (4, 3, 7)
    s = -1.0 if code & 0x80 else 1.0
    e, m = (code >> mb) & ((1 << eb) - 1), code & ((1 << mb) - 1)
    if e == (1 << eb) - 1:
        if e5m2:
            return s * math.inf if m == 0 else math.nan
        if m == (1 << mb) - 1:
            return math.nan
    if e == 0:
        return s * m / (1 << mb) * 2.0 ** (1 - bias)
    return s * (1 + m / (1 << mb)) * 2.0 ** (e - bias)


@pytest.mark.parametrize("e5m2", [False, True])
def test_fp8_decode_matches_the_format_for_every_code(orc, e5m2):
    for code in range(256):
        a, b = orc.fp8_decode(e5m2, code), fp8_value(e5m2, code)
        assert (math.isnan(a) and math.isnan(b)) or a == b, (code, a, b)


def test_fp8_published_values_and_rounding(orc):
    """fp8/tests.rs:3-58"""
    d = lambda c: orc.fp8_decode(False, c)
    assert d(0x00) == 0.0 and d(0x01) == 2.0 ** -9 and d(0x08) == 2.0 ** -6 and d(0x38) == 1.0
    assert d(0x7e) == 448.0 and math.isnan(d(0x7f)) and math.isnan(d(0xff)) and d(0xb8) == -1.0
    e = lambda c: orc.fp8_decode(True, c)
    assert e(0x01) == 2.0 ** -16 and e(0x04) == 2.0 ** -14 and e(0x3c) == 1.0 and e(0x7b) == 57344.0
    assert e(0x7c) == math.inf and e(0xfc) == -math.inf and math.isnan(e(0x7d))
    enc = lambda x: orc.fp8_encode(False, x)
    assert enc(1.0625) == 0x38 and enc(1.0626) == 0x39 and enc(1.1875) == 0x3A
    assert enc(1.0e9) == 0x7E and enc(-1.0e9) == 0xFE and enc(math.inf) == 0x7E and enc(-0.0) == 0x80
    assert enc(math.nan) == 0x7F and orc.fp8_encode(True, math.nan) == 0x7E and orc.fp8_encode(True, 1.0e9) == 0x7B


@pytest.mark.parametrize("e5m2", [False, True])
def test_fp8_encode_is_the_nearest_code_with_ties_to_even(orc, e5m2):
    """Against an exhaustive search over the finite codes (a different algorithm from the
    reference's binary search), on random values, midpoints and every code's value."""
    limit = 0x7B if e5m2 else 0x7E
    vals = np.array([fp8_value(e5m2, c) for c in range(limit + 1)])
    xs = list(vals) + list((vals[1:] + vals[:-1]) / 2)
    rng = np.random.default_rng(3)
    xs += list(rng.uniform(0, vals[-1] * 1.2, 3000)) + list(rng.uniform(0, 2 * vals[8], 1000))
    for x in xs:
        x = float(np.float32(x))
        for s in (x, -x):
            got = orc.fp8_encode(e5m2, s)
            a = min(abs(s), vals[-1])
            dist = np.abs(vals - a)
            best = np.flatnonzero(dist == dist.min())
            pick = int(best[0]) if len(best) == 1 else int(best[best % 2 == 0][0])
            assert got == (0x80 if math.copysign(1, s) < 0 else 0) | pick, (s, got, pick)


@pytest.mark.parametrize("ty,tol", [("FP8_E4M3", 0.07), ("FP8_E5M2", 0.13)])
def test_fp8_blocks_scale_to_the_range(orc, ty, tol):
    """fp8/tests.rs:61-80"""
    t = getattr(orc, ty)
    data = np.array([math.sin(i * 0.31) * (1 + i % 5) for i in range(64)], np.float32)
    b = orc.encode(t, data)
    assert b.size == 68
    back = orc.decode(t, b, 64)
    for blk, got in zip(data.reshape(2, 32), back.reshape(2, 32)):
        assert np.all(np.abs(blk - got) <= tol * np.abs(blk).max())
    assert np.array_equal(orc.decode(t, orc.encode(t, np.zeros(32)), 32), np.zeros(32))


# ---- MXFP4 ----

def test_mxfp4_half_scale_and_known_blocks(orc):
    """mxfp4/tests.rs:3-74"""
    for e in range(255):
        assert orc.mxfp4_half_scale(e) == np.float32(2.0 ** (e - 128)), e
    vals_ = [0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12]
    vals = np.array([vals_[i % 16] * 0.5 for i in range(32)], np.float32)
    b = orc.encode(orc.MXFP4, vals)
    assert b.size == 17 and b[0] == 127 and b[1] & 15 == 0 and b[2] & 15 == 1
    assert np.array_equal(orc.decode(orc.MXFP4, b, 32), vals)
    data = np.array([((i * 37 % 101) - 50.0) / 25.0 for i in range(64)], np.float32)
    back = orc.decode(orc.MXFP4, orc.encode(orc.MXFP4, data), 64)
    for blk, got in zip(data.reshape(2, 32), back.reshape(2, 32)):
        amax = np.abs(blk).max()
        d = orc.mxfp4_half_scale(int(np.floor(np.log2(amax))) - 2 + 127)
        for x, y in zip(blk, got):
            limit = 2 * d if abs(x) <= 12 * d else abs(x) - 12 * d
            assert abs(x - y) <= limit + 1e-6
    assert list(orc.encode(orc.MXFP4, np.zeros(32))) == [0] * 17
    v = np.full(32, 0.5, np.float32)
    v[3] = np.inf
    assert orc.encode(orc.MXFP4, v)[0] == 0
    assert orc.encode(orc.MXFP4, np.full(32, 3.0e38, np.float32))[0] == 252
    assert np.all(np.isfinite(orc.decode(orc.MXFP4, orc.encode(orc.MXFP4, np.full(32, 1e-38, np.float32)), 32)))
    t = np.zeros(32, np.float32)
    t[0], t[1] = 6.0, 2.5
    b = orc.encode(orc.MXFP4, t)
    assert b[1] & 15 == 7 and b[1] >> 4 == 0 and b[2] & 15 == 4


def test_mxfp4_scale_byte_near_powers_of_two(orc):
    """The scale byte is floor(log2(amax)) - 2 + 127 with glibc's log2f (what Rust's f32::log2
    calls): checked against float64 log2 rounded to f32 on the floats nearest every power of
    two, where a log2 that rounds up would move the scale (the device computes it that way)."""
    for k in range(-120, 127):
        p = np.float32(2.0 ** k)
        for x in (np.nextafter(p, np.float32(0)), p, np.nextafter(p, np.float32(np.inf))):
            blk = np.zeros(32, np.float32)
            blk[0] = x
            want = int(math.floor(float(np.float32(math.log2(float(x)))))) - 2 + 127
            assert orc.encode(orc.MXFP4, blk)[0] == min(max(want, 0), 254), (k, x)


# ---- Q2_K ----

def q2k_decode_np(b: np.ndarray) -> np.ndarray:
    """Q2_K from the ggml layout, written independently: scales[16] (low nibble scale, high nibble
    min), qs[64] (2-bit fields: element 32 s + l of half h at bit 2 s of byte 32 h + l), d, dmin."""
    out = []
    for blk in b.reshape(-1, 84):
        sc, qs = blk[:16], blk[16:80]
        d = float(np.frombuffer(blk[80:82].tobytes(), np.float16)[0])
        dm = float(np.frombuffer(blk[82:84].tobytes(), np.float16)[0])
        vals = np.zeros(256)
        for i in range(256):
            h, r = divmod(i, 128)
            s, l = divmod(r, 32)
            q = (int(qs[32 * h + l]) >> (2 * s)) & 3
            sub = i // 16
            vals[i] = np.float32(np.float32(d) * np.float32(sc[sub] & 15)) * np.float32(q) - \
                np.float32(np.float32(dm) * np.float32(sc[sub] >> 4))
        out.append(vals)
    return np.concatenate(out).astype(np.float32)


def wave(n):
    return np.array([math.sin(i * 0.37) * 0.8 + ((i * 7 % 13) - 6.0) * 0.02 for i in range(n)], np.float32)


def test_q2k_known_answers_and_properties(orc):
    """q2k/tests.rs:16-84"""
    for x, want in [(0.5, 0), (1.5, 2), (2.5, 2), (-0.5, 0), (-1.5, -2), (3.7, 4), (-3.7, -4), (0.0, 0)]:
        assert orc.q2k_nearest_int(x) == want
    data = wave(1024)
    b = orc.encode(orc.Q2_K, data)
    assert b.size == 4 * 84
    back = orc.decode(orc.Q2_K, b, 1024)
    assert np.array_equal(back, q2k_decode_np(b))
    signal = np.sqrt((data ** 2).mean())
    assert np.sqrt(((data - back) ** 2).mean()) < 0.30 * signal
    for sub, got in zip(data.reshape(-1, 16), back.reshape(-1, 16)):
        assert np.all(np.abs(sub - got) <= (sub.max() - sub.min()) / 3 + 0.02)
    z = orc.encode(orc.Q2_K, np.zeros(256))
    assert not z.any() and not orc.decode(orc.Q2_K, z, 256).any()
    assert np.all(np.abs(orc.decode(orc.Q2_K, orc.encode(orc.Q2_K, np.full(256, 0.5)), 256) - 0.5) < 0.2)
    assert np.all(np.abs(orc.decode(orc.Q2_K, orc.encode(orc.Q2_K, np.full(256, -0.5)), 256) + 0.5) < 0.05)
    w = wave(512)
    a = orc.encode(orc.Q2_K, w)
    assert np.array_equal(a, orc.encode(orc.Q2_K, w))
    assert np.array_equal(a[:84], orc.encode(orc.Q2_K, w[:256])) and np.array_equal(a[84:], orc.encode(orc.Q2_K, w[256:]))


def q2k_nearest_int_np(x):
    """ggml's nearest_int: (x + 1.5 * 2^23) in f32, then the low 23 bits minus 2^22."""
    return ((np.asarray(x, np.float32) + np.float32(12582912.0)).view(np.int32) & 0x7FFFFF) - 0x400000


def seqsum(a):
    """Left-to-right f32 sum along the last axis (0 + a0 + a1 + ...)."""
    return np.cumsum(a, axis=-1, dtype=np.float32)[..., -1]


def q2k_fit_np(x, rmin=-0.5, rdelta=0.1, nstep=15, clamp_min=True, moving_min=True, unit_weights=False,
               keep_worse=False):
    """make_qkx2_quants for nmax = 3 over sub-blocks x [S, 16]: the scale and (negated) min of the
    candidate grid point whose weighted (|x|) absolute deviation is smallest, first wins (each
    candidate's grid spans max - min with the min of the best candidate so far); the quants of
    that candidate."""
    f = np.float32
    x = np.asarray(x, f)
    w = np.ones_like(x) if unit_weights else np.abs(x)
    mn, mx = x.min(axis=1), x.max(axis=1)
    sum_w, sum_x = seqsum(w), seqsum(w * x)
    mn = np.where(mn > 0, f(0), mn)
    mn0 = mn
    flat = mx == mn
    with np.errstate(all="ignore"):
        rng = mx - mn
        iscale = f(3) / rng
        scale = f(1) / iscale
        lv = np.clip(q2k_nearest_int_np(iscale[:, None] * (x - mn[:, None])), 0, 3)
        best = seqsum(w * np.abs(scale[:, None] * lv.astype(f) + mn[:, None] - x))
        for step in range(nstep + 1):  # a taken candidate's min moves the grid of the later ones
            lo = mn if moving_min else mn0
            isc = (f(rmin) + f(rdelta) * f(step) + f(3)) / (mx - lo)
            la = np.clip(q2k_nearest_int_np(isc[:, None] * (x - lo[:, None])), 0, 3)
            qf = la.astype(f)
            sl, sl2, sxl = seqsum(w * qf), seqsum(w * qf * qf), seqsum(w * qf * x)
            d = sum_w * sl2 - sl * sl
            ts = (sum_w * sxl - sum_x * sl) / d
            tm = (sl2 * sum_x - sl * sxl) / d
            if clamp_min:
                pos = tm > 0
                tm = np.where(pos, f(0), tm)
                ts = np.where(pos, sxl / sl2, ts)
            mad = seqsum(w * np.abs(ts[:, None] * qf + tm[:, None] - x))
            take = (d > 0) & ((mad > best) if keep_worse else (mad < best)) & ~flat
            lv = np.where(take[:, None], la, lv)
            best = np.where(take, mad, best)
            scale = np.where(take, ts, scale)
            mn = np.where(take, tm, mn)
    lv = np.where(flat[:, None], 0, lv)
    scale = np.where(flat, f(0), scale)
    return scale.astype(f), (-mn).astype(f), lv


def q2k_encode_np(data, requant=True, **search):
    """Q2_K super-blocks from q2k_fit_np: 4-bit scales and mins against the f16 super scale and
    min, the quants re-fitted to the rounded scales, then the ggml layout."""
    f = np.float32
    blocks = np.asarray(data, f).reshape(-1, 256)
    sc, mins, lv = q2k_fit_np(blocks.reshape(-1, 16), **search)
    sc, mins, lv = sc.reshape(-1, 16), mins.reshape(-1, 16), lv.reshape(-1, 256)
    out = []
    for b in range(blocks.shape[0]):
        ms, mm = max(f(0), sc[b].max()), max(f(0), mins[b].max())
        packed = np.zeros(16, np.int64)
        dbits = mbits = 0
        if ms > 0:
            packed = q2k_nearest_int_np((f(15) / ms) * sc[b]).astype(np.int64) & 0xFF
            dbits = int(np.float32(ms / f(15)).astype(np.float16).view(np.uint16))
        if mm > 0:
            packed |= ((q2k_nearest_int_np((f(15) / mm) * mins[b]).astype(np.int64) & 0xFF) << 4) & 0xFF
            mbits = int(np.float32(mm / f(15)).astype(np.float16).view(np.uint16))
        d32 = np.array(dbits, np.uint16).view(np.float16).astype(f)
        m32 = np.array(mbits, np.uint16).view(np.float16).astype(f)
        levels = lv[b].copy()
        for j in range(16 if requant else 0):
            s_ = d32 * f(packed[j] & 15)
            if s_ == 0:
                continue
            dm = m32 * f(packed[j] >> 4)
            levels[16 * j:16 * j + 16] = np.clip(q2k_nearest_int_np((blocks[b, 16 * j:16 * j + 16] + dm) / s_), 0, 3)
        qs = []
        for half in (0, 128):
            for l in range(32):
                qs.append(levels[half + l] | levels[half + l + 32] << 2 | levels[half + l + 64] << 4 |
                          levels[half + l + 96] << 6)
        out.append(np.concatenate([packed.astype(np.uint8), np.array(qs, np.uint8),
                                   np.array([dbits & 0xFF, dbits >> 8, mbits & 0xFF, mbits >> 8], np.uint8)]))
    return np.concatenate(out)


def q2k_cases():
    """Data that reaches every branch of the search: smooth and noisy signals, all-positive
    sub-blocks (min clamped to zero), all-negative ones, flat sub-blocks, lone spikes, magnitudes
    from 1e-6 to 1e3 side by side, and scales small enough to round to f16 subnormals."""
    rng = np.random.default_rng(21)
    cases = {"wave": wave(4096), "normal": (rng.standard_normal(16384) * 0.02).astype(np.float32),
             "heavy": rng.standard_t(2, 8192).astype(np.float32),
             "positive": np.abs(rng.standard_normal(4096)).astype(np.float32) + np.float32(0.1),
             "negative": -np.abs(rng.standard_normal(4096)).astype(np.float32)}
    mixed = rng.standard_normal(8192).astype(np.float32)
    mixed *= np.float32(10.0) ** rng.integers(-6, 4, 8192 // 16).repeat(16).astype(np.float32)
    cases["mixed"] = mixed
    spiky = np.zeros(4096, np.float32)
    spiky[rng.integers(0, 4096, 64)] = rng.standard_normal(64).astype(np.float32)
    cases["spiky"] = spiky
    flat = rng.standard_normal(4096).astype(np.float32)
    flat[: 2048] = np.repeat(rng.standard_normal(128).astype(np.float32), 16)
    cases["flat"] = flat
    cases["tiny"] = (rng.standard_normal(2048) * 1e-7).astype(np.float32)
    return cases


@pytest.mark.parametrize("name", list(q2k_cases()))
def test_q2k_encoder_equals_an_independent_numpy_search(orc, name):
    data = q2k_cases()[name]
    assert np.array_equal(orc.encode(orc.Q2_K, data), q2k_encode_np(data)), name


def test_q2k_search_constants_are_pinned_by_the_cases(orc):
    """Each perturbation of the search changes some case's bytes, so the match above pins them."""
    cases = q2k_cases()
    want = {n: orc.encode(orc.Q2_K, d) for n, d in cases.items()}
    for bad in ({"rmin": -0.4}, {"rdelta": 0.11}, {"nstep": 14}, {"clamp_min": False}, {"moving_min": False}):
        assert any(not np.array_equal(want[n], q2k_encode_np(d, **bad)) for n, d in cases.items()), bad


# ---- Q2_K pinned by what the mathematics fixes, not by a second statement of the search ----

def q2k_fit_violations(x, scale, neg_min, levels):
    """Sub-blocks [S, 16] whose (scale, min, levels) break what make_qkx2_quants promises
    (q2k.rs:24-93), judged in float64 from the definitions alone:
    - a flat sub-block (max == min) gets scale 0 and levels 0;
    - otherwise (scale, min) is either the first candidate, the grid spanning [min(x, 0), max]
      (scale (max - min) / 3), or the |x|-weighted least-squares fit of x by scale * l + min over
      the returned levels, with the min clamped to 0 (and the scale refitted) when the fit's min
      is positive, to 1e-4 of the grid step (f32 sums of 16 terms);
    - its |x|-weighted absolute deviation is no larger than the first candidate's (up to the f32
      rounding of the scale and min).
    Returns the indices of the failing sub-blocks."""
    x = np.asarray(x, np.float64)
    s = np.asarray(scale, np.float64)
    m = -np.asarray(neg_min, np.float64)
    lq = np.asarray(levels, np.float64)
    bad = []
    for i in range(x.shape[0]):
        xi, li = x[i], lq[i]
        mn, mx = min(xi.min(), 0.0), xi.max()
        if mx == mn:
            if s[i] != 0 or li.any():
                bad.append(i)
            continue
        step = (mx - mn) / 3
        w = np.abs(xi)
        first_l = np.clip(np.rint((xi - mn) / step), 0, 3)
        first_mad = np.sum(w * np.abs(step * first_l + mn - xi))
        is_first = abs(s[i] - step) <= 1e-6 * step and abs(m[i] - mn) <= 1e-6 * step
        if not is_first:
            sw, sx, sl = w.sum(), (w * xi).sum(), (w * li).sum()
            sl2, sxl = (w * li * li).sum(), (w * li * xi).sum()
            det = sw * sl2 - sl * sl
            if det <= 0:
                bad.append(i)
                continue
            fs, fm = (sw * sxl - sx * sl) / det, (sl2 * sx - sl * sxl) / det
            if fm > 0:
                fs, fm = sxl / sl2, 0.0
            if abs(s[i] - fs) > 1e-4 * step or abs(m[i] - fm) > 1e-4 * step:
                bad.append(i)
                continue
        mad = np.sum(w * np.abs(s[i] * li + m[i] - xi))
        if mad > first_mad * (1 + 1e-5) + 1e-6 * w.sum() * step:  # f32 scale and min roundings
            bad.append(i)
    return bad


def q2k_block_violations(data, blob, scale, neg_min):
    """Super-blocks whose bytes break the packing rules (q2k.rs:96-150), in float64: the 4-bit
    scale (min) codes are the nearest integers to 15 * scale_j / max_scale (min_j / max_min), the
    f16 super scale is max_scale / 15 rounded to f16, and every level is the nearest of 0..3 to
    (x + dmin * m_j) / (d * s_j), the decoder's own sub-block scale and min (clamped at the ends),
    wherever that scale is not 0."""
    x = np.asarray(data, np.float64).reshape(-1, 256)
    raw = np.asarray(blob, np.uint8).reshape(-1, 84)
    sc, mi = np.asarray(scale, np.float64).reshape(-1, 16), np.asarray(neg_min, np.float64).reshape(-1, 16)
    bad = []
    for b in range(x.shape[0]):
        codes = raw[b, :16]
        d = float(raw[b, 80:82].copy().view(np.float16)[0])
        dmin = float(raw[b, 82:84].copy().view(np.float16)[0])
        ok = True
        for vals, nib, sup in ((sc[b], codes & 15, d), (mi[b], codes >> 4, dmin)):
            top = max(0.0, vals.max())
            if top > 0:
                ok &= bool(np.all(np.abs(15 * vals / top - nib) <= 0.5 + 1e-6))
                ok &= float(np.float16(np.float32(top / 15))) == sup
            else:
                ok &= bool(np.all(nib == 0)) and sup == 0
        q = raw[b, 16:80]
        lv = np.empty(256, np.int64)
        for h in range(2):
            for j in range(4):
                lv[128 * h + 32 * j:128 * h + 32 * j + 32] = (q[32 * h:32 * h + 32] >> (2 * j)) & 3
        for j in range(16):
            s_ = d * float(codes[j] & 15)
            if s_ == 0:
                continue
            t = (x[b, 16 * j:16 * j + 16] + dmin * float(codes[j] >> 4)) / s_
            L = lv[16 * j:16 * j + 16]
            near = np.abs(t - L) <= 0.5 + 1e-6 * np.maximum(1, np.abs(t))
            ok &= bool(np.all(near | ((L == 0) & (t < 0)) | ((L == 3) & (t > 3))))
        if not ok:
            bad.append(b)
    return bad


def oracle_q2k_fits(orc, data):
    subs = np.asarray(data, np.float32).reshape(-1, 16)
    out = [orc.q2k_fit(s) for s in subs]
    return (subs, np.array([o[0] for o in out], np.float32), np.array([o[1] for o in out], np.float32),
            np.stack([o[2] for o in out]))


@pytest.mark.parametrize("name", list(q2k_cases()))
def test_q2k_oracle_meets_the_least_squares_and_packing_rules(orc, name):
    data = q2k_cases()[name]
    subs, sc, mn, lv = oracle_q2k_fits(orc, data)
    assert q2k_fit_violations(subs, sc, mn, lv) == [], name
    assert q2k_block_violations(data, orc.encode(orc.Q2_K, data), sc, mn) == [], name


def test_q2k_rules_catch_planted_mistakes(orc):
    """Misreadings that a second statement of the search could share, each planted in the numpy
    restatement: the fit unweighted (w = 1), the worse candidate kept, the min clamp dropped, the
    min's sign flipped, and the levels left on the search grid instead of re-fitted to the rounded
    scales. Each breaks the rules above on the cases."""
    cases = q2k_cases()
    both = np.concatenate([cases["normal"], cases["heavy"], cases["positive"], cases["mixed"]])
    subs = both.reshape(-1, 16)
    for bad in ({"unit_weights": True}, {"keep_worse": True}, {"clamp_min": False}):
        sc, mn, lv = q2k_fit_np(subs, **bad)
        assert len(q2k_fit_violations(subs, sc, mn, lv)) > 0, bad
    sc, mn, lv = q2k_fit_np(subs)
    assert q2k_fit_violations(subs, sc, mn, lv) == []
    assert len(q2k_fit_violations(subs, sc, -mn, lv)) > 0
    blob = q2k_encode_np(both, requant=False)
    assert len(q2k_block_violations(both, blob, sc, mn)) > 0
    assert q2k_block_violations(both, q2k_encode_np(both), sc, mn) == []


# ---- read-only block types (blocks/tests.rs) ----

def test_block_layouts_and_known_blocks(orc):
    for ty, nb, ne in [(orc.Q4_1, 20, 32), (orc.Q5_0, 22, 32), (orc.Q5_1, 24, 32), (orc.Q8_1, 36, 32),
                       (orc.Q2_K, 84, 256), (orc.Q3_K, 110, 256), (orc.Q4_K, 144, 256), (orc.Q5_K, 176, 256),
                       (orc.Q6_K, 210, 256)]:
        assert orc.nbytes(ty, 2 * ne) == 2 * nb and orc.nbytes(ty, ne + 1) == -1
        assert orc.decode(ty, np.zeros(2 * nb, np.uint8), 2 * ne).size == 2 * ne
        if ty != orc.Q2_K:  # read-only: loaded, never written (quant.rs:92-96)
            with pytest.raises(ValueError, match="read-only"):
                orc.encode(ty, np.zeros(ne))
    close = lambda a, b: abs(a - b) < 1e-3
    raw = np.array(f16b(0.5) + f16b(7.0) + [(i - 16) & 0xFF for i in range(32)], np.uint8)
    assert all(close(v, 0.5 * (i - 16)) for i, v in enumerate(orc.decode(orc.Q8_1, raw, 32)))
    los, his = [j % 15 for j in range(16)], [(j + 3) % 15 for j in range(16)]
    raw = np.array(f16b(0.25) + f16b(1.0) + [(his[j] << 4) | los[j] for j in range(16)], np.uint8)
    out = orc.decode(orc.Q4_1, raw, 32)
    assert all(close(out[j], 0.25 * los[j] + 1) and close(out[j + 16], 0.25 * his[j] + 1) for j in range(16))
    qh = 1 | (1 << 17)
    raw = f16b(2.0) + list(qh.to_bytes(4, "little")) + [0x21] * 16
    q = orc.decode(orc.Q5_0, np.array(raw, np.uint8), 32)
    assert (q[0], q[1], q[17], q[16]) == (2.0, -30.0, 4.0, -28.0)
    raw = raw[:2] + f16b(0.5) + raw[2:]
    q = orc.decode(orc.Q5_1, np.array(raw, np.uint8), 32)
    assert (q[0], q[17], q[1]) == (34.5, 36.5, 2.5)
    sc = [2, 2, 2, 2, 0, 0, 0, 0, 2, 2, 2, 2]
    raw = np.array(f16b(0.5) + f16b(0.0) + sc + [0x33] * 128, np.uint8)
    assert all(close(v, 3.0) for v in orc.decode(orc.Q4_K, raw, 256))
    raw = np.array(f16b(1.0) + f16b(0.5) + [2, 2, 2, 2, 1, 1, 1, 1, 0x12, 0x12, 0x12, 0x12] + [0x75] * 128, np.uint8)
    out = orc.decode(orc.Q4_K, raw, 256)
    assert close(out[0], 9.5) and close(out[32], 13.5) and close(out[128], 9.5) and close(out[160], 13.5)
    for qhb, want in ((0, 3.0), (0xFF, 19.0)):
        raw = np.array(f16b(0.5) + f16b(0.0) + sc + [qhb] * 32 + [0x33] * 128, np.uint8)
        assert all(close(v, want) for v in orc.decode(orc.Q5_K, raw, 256))
    raw = np.array([0x88] * 128 + [0xAA] * 64 + [2] * 16 + f16b(0.5), np.uint8)
    assert all(close(v, 8.0) for v in orc.decode(orc.Q6_K, raw, 256))
    raw = np.array([0x88] * 128 + [0xAA] * 64 + [(i - 8) & 0xFF for i in range(16)] + f16b(1.0), np.uint8)
    out = orc.decode(orc.Q6_K, raw, 256)
    assert close(out[0], -64) and close(out[16], -56) and close(out[32], -48) and close(out[128], 0)
    b = np.zeros(84, np.uint8)
    b[:16] = [i | ((15 - i) << 4) for i in range(16)]
    b[16:80] = 0x55
    b[80:82], b[82:84] = f16b(1.0), f16b(0.5)
    for g, chunk in enumerate(orc.decode(orc.Q2_K, b, 256).reshape(16, 16)):
        assert all(close(v, g - 0.5 * (15 - g)) for v in chunk)
    b = np.zeros(110, np.uint8)
    b[32:96], b[96:104], b[104:108], b[108:110] = 0x55, 0x22, 0xAA, f16b(1.0)
    b[:32] = 0xFF
    assert all(close(v, 2.0) for v in orc.decode(orc.Q3_K, b, 256))
    b[:32] = 0
    assert all(close(v, -6.0) for v in orc.decode(orc.Q3_K, b, 256))


def test_quantise_matrix_takes_the_new_formats(orc):
    rng = np.random.default_rng(4)
    for ty, k in ((orc.MXFP4, 64), (orc.FP8_E4M3, 64), (orc.FP8_E5M2, 96), (orc.Q2_K, 256), (orc.F16, 32)):
        w = rng.standard_normal(k * 3).astype(np.float32)
        b = orc.quantise_matrix(ty, w, k, 3)
        assert np.array_equal(b, orc.encode(ty, orc.transpose(w, k, 3)))
    with pytest.raises(ValueError):
        orc.quantise_matrix(orc.Q2_K, np.zeros(96), 96, 1)
