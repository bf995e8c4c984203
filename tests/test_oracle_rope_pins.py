"""CPU pins of the RoPE parts of the prologue oracle that the reference's
tiny goldens do not reach: the vision tower's axial RoPE and its tables, the
Qwen3.5 partial RoPE, and both table constructions (f64 angles, and the f32
angles of Qwen3.5 and the vision tower).

Each pin is an independent statement of the answer, chosen so that a
plausible mistake fails it:
- the reference's own equivalence test for the axial rotation
  (crates/inl-vision/src/vision.rs:974-1041), restated with its LCG inputs:
  concatenated ``[cos_x, cos_x, cos_y, cos_y]`` tables and two half-split
  rotations of its ``reference_rotary`` spelling;
- invariants of the partial rotation (crates/inl-late/src/qwen3_5.rs:289-300);
- closed forms of the tables in f64, within a stated f32 error bound
  (qwen3_5.rs:940-957, vision.rs:760-780, qwen3/mod.rs:131-153).
Planted mistakes (swapped halves, interleaved pairs, a wrong theta exponent,
the rotation over the whole head) are shown to fail the same checks.
"""
import numpy as np

from oracle import prologue as op

U64 = (1 << 64) - 1


def ramp(n, seed):
    """The vision tests' LCG (crates/inl-vision/src/vision.rs:927-937): u64
    wrapping state, values ``(state >> 40) / 2^23 - 1`` in [-1, 1), f32."""
    a, c = 6364136223846793005, 1442695040888963407
    state = (seed * 2_654_435_761 + 1) & U64
    out = np.empty(n, dtype=np.float32)
    for i in range(n):
        state = (state * a + c) & U64
        out[i] = np.float32(state >> 40) / np.float32(1 << 23) - np.float32(1.0)
    return out


def reference_rotary(x, cos, sin):
    """vision.rs:976-982: ``x * cos + cat(-b, a) * sin`` over the last axis,
    with full-width ``cos``/``sin``."""
    half = x.shape[-1] // 2
    rotated = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    return x * cos + rotated * sin


def reference_axial_rope(x, cos, sin):
    """vision.rs:984-996: x ``[b, t, h, d]``, tables ``[b, t, d]`` laid out
    ``[cos_x, cos_x, cos_y, cos_y]``; each head half is rotated by its half of
    the tables."""
    part = x.shape[-1] // 2
    c0, s0 = cos[:, :, None, :part], sin[:, :, None, :part]
    c1, s1 = cos[:, :, None, part:], sin[:, :, None, part:]
    y0 = reference_rotary(x[..., :part], c0, s0)
    y1 = reference_rotary(x[..., part:], c1, s1)
    return np.concatenate([y0, y1], axis=-1)


def _vision_case():
    """vision.rs:1001-1017: batch 2, seq 5, heads 2, head_dim 64 (the test
    config), rope_theta 100, positions round(4 * ramp(., 7)), x = ramp(., 11)."""
    batch, seq, heads, dim, theta = 2, 5, 2, 64, 100.0
    pos = np.round(ramp(batch * seq * 2, 7) * np.float32(4.0)).astype(np.float32)
    pos = pos.reshape(batch, seq, 2)
    x = ramp(batch * seq * heads * dim, 11).reshape(batch, seq, heads, dim).astype(np.float64)
    return pos, x, dim, theta


def _oracle_axial(pos, x, dim, theta, swap=False):
    inv = op.vision_inv_freq(dim, theta)
    b, t = pos.shape[:2]
    cx, sx, cy, sy = op.axial_tables(inv, pos.reshape(b * t, 2))
    if swap:
        cx, sx, cy, sy = cy, sy, cx, sx
    y = op.axial_rope(x.reshape(b * t, x.shape[2], dim), cx, sx, cy, sy)
    return y.reshape(x.shape), (cx, sx, cy, sy)


def test_axial_rope_matches_the_reference_spelling():
    pos, x, dim, theta = _vision_case()
    got, (cx, sx, cy, sy) = _oracle_axial(pos, x, dim, theta)
    b, t = pos.shape[:2]
    cos = np.concatenate([cx, cx, cy, cy], axis=1).reshape(b, t, dim).astype(np.float64)
    sin = np.concatenate([sx, sx, sy, sy], axis=1).reshape(b, t, dim).astype(np.float64)
    want = reference_axial_rope(x, cos, sin)
    # the reference's f32 bound is 1e-4; both sides here are f64 over the same
    # f32 tables, so they agree to rounding
    assert np.abs(got - want).max() < 1e-12
    # the positions are not all equal and not all zero, so the check rotates
    assert np.abs(got - x).max() > 0.1


def test_axial_rope_planted_mistakes_fail():
    pos, x, dim, theta = _vision_case()
    good, (cx, sx, cy, sy) = _oracle_axial(pos, x, dim, theta)
    b, t = pos.shape[:2]
    cos = np.concatenate([cx, cx, cy, cy], axis=1).reshape(b, t, dim).astype(np.float64)
    sin = np.concatenate([sx, sx, sy, sy], axis=1).reshape(b, t, dim).astype(np.float64)
    want = reference_axial_rope(x, cos, sin)
    # x and y tables swapped between the head halves
    swapped, _ = _oracle_axial(pos, x, dim, theta, swap=True)
    assert np.abs(swapped - want).max() > 1e-2
    # one half-split over the whole head with the x tables only
    whole = op.rope(x.reshape(b * t, 2, dim), np.concatenate([cx, cx], 1)[:, None, :],
                    np.concatenate([sx, sx], 1)[:, None, :]).reshape(x.shape)
    assert np.abs(whole - want).max() > 1e-2
    # interleaved pairs (2i, 2i+1) instead of the half split inside each half
    xi = x.reshape(b * t, 2, dim)
    inter = xi.copy()
    half = dim // 2
    for h0, (c, s) in ((0, (cx, sx)), (half, (cy, sy))):
        e, o = xi[..., h0:h0 + half:2], xi[..., h0 + 1:h0 + half:2]   # dim/4 pairs per half
        cc, ss = c[:, None, :], s[:, None, :]
        inter[..., h0:h0 + half:2] = e * cc - o * ss
        inter[..., h0 + 1:h0 + half:2] = o * cc + e * ss
    assert np.abs(inter.reshape(x.shape) - want).max() > 1e-2


def test_vision_inv_freq_closed_form():
    """``1 / theta^(2i / spatial)`` with spatial = head_dim / 2, head_dim/4
    entries (vision.rs:760-767), within 4 f32 ulps of the f64 value; the
    exponent over head_dim instead of spatial is far outside that bound."""
    for dim, theta in ((64, 100.0), (64, 10000.0), (128, 100.0)):
        got = op.vision_inv_freq(dim, theta).astype(np.float64)
        spatial = dim // 2
        i = np.arange(spatial // 2)
        want = 1.0 / np.power(theta, 2.0 * i / spatial)
        assert got.shape == (dim // 4,)
        assert np.all(np.abs(got - want) <= 4 * 2.0 ** -24 * want)
        wrong = 1.0 / np.power(theta, 2.0 * i / dim)
        assert np.abs(wrong - want).max() > 1e-2


def test_axial_tables_closed_form():
    """cos/sin of position * inv_freq per axis (vision.rs:771-780): column 0
    of the positions drives the x tables, column 1 the y tables; within the
    f32 rounding of the product and of cos/sin."""
    rng = np.random.default_rng(3)
    dim, theta = 64, 100.0
    pos = rng.integers(0, 48, size=(300, 2)).astype(np.float32)
    inv32 = op.vision_inv_freq(dim, theta)
    cx, sx, cy, sy = op.axial_tables(inv32, pos)
    inv = inv32.astype(np.float64)
    for c, s, col in ((cx, sx, 0), (cy, sy, 1)):
        ang = pos[:, col:col + 1].astype(np.float64) * inv[None, :]
        bound = np.abs(ang) * 2.0 ** -23 + 2.0 ** -23
        assert np.all(np.abs(c - np.cos(ang)) <= bound)
        assert np.all(np.abs(s - np.sin(ang)) <= bound)
    # the axes are distinct in this sample, so a swap would show
    assert np.abs(cx - cy).max() > 0.5


def test_partial_rope_invariants():
    """qwen3_5.rs:289-300: the first rotary_dim features are the half-split
    rotation of that slice (its pairs are (i, i + rotary_dim/2), not
    (i, i + head_dim/2)), the rest pass through unchanged, and every rotated
    pair keeps its norm."""
    rng = np.random.default_rng(5)
    hd, rd, n = 256, 64, 40
    c, s = op.rope_table_f32(rd, 1e7, n)
    c, s = c.astype(np.float64)[:, None, :], s.astype(np.float64)[:, None, :]
    x = rng.standard_normal((n, 3, hd))
    y = op.partial_rope(x, c, s, rd)
    assert np.array_equal(y[..., rd:], x[..., rd:])
    # the reference's test spelling of the half-split on the slice
    want = op.rope_manual(x[..., :rd], c, s)
    assert np.abs(y[..., :rd] - want).max() < 1e-12
    h = rd // 2
    assert np.allclose(x[..., :h] ** 2 + x[..., h:rd] ** 2, y[..., :h] ** 2 + y[..., h:rd] ** 2)
    # planted: pairs (i, i + head_dim/2) over the whole head
    cw = np.concatenate([c, np.ones((n, 1, hd // 2 - rd // 2))], -1)
    sw = np.concatenate([s, np.zeros((n, 1, hd // 2 - rd // 2))], -1)
    wrong = op.rope(x, cw, sw)
    assert np.abs(wrong[..., :rd] - y[..., :rd]).max() > 1e-2
    # rotary_dim == head_dim is the plain rope
    cf, sf = op.rope_table_f32(hd, 1e7, n)
    cf, sf = cf.astype(np.float64)[:, None, :], sf.astype(np.float64)[:, None, :]
    assert np.abs(op.partial_rope(x, cf, sf, hd) - op.rope(x, cf, sf)).max() == 0.0


def test_rope_table_f32_closed_form():
    """Qwen3.5 tables (qwen3_5.rs:940-957): inv_freq = 1 / theta^(2i/dim) and
    the position products in f32. Against the f64 closed form the error is at
    most the f32 rounding of inv_freq (powf and the division, 4 ulps), of the
    product (half an ulp of the angle) and of cos/sin (one ulp): bound
    |angle| * 2^-21 + 2^-23. A wrong exponent (2i / (dim/2)) or a table over
    the full head instead of rotary_dim fails it."""
    for dim, theta, n in ((64, 1e7, 300), (32, 1e4, 64), (128, 1e6, 500)):
        c, s = op.rope_table_f32(dim, theta, n)
        assert c.dtype == np.float32 and c.shape == (n, dim // 2)
        i = np.arange(dim // 2)
        ang = np.arange(n, dtype=np.float64)[:, None] / np.power(theta, 2.0 * i / dim)[None, :]
        bound = np.abs(ang) * 2.0 ** -21 + 2.0 ** -23
        assert np.all(np.abs(c - np.cos(ang)) <= bound)
        assert np.all(np.abs(s - np.sin(ang)) <= bound)
        wrong = np.arange(n, dtype=np.float64)[:, None] / np.power(theta, 4.0 * i / dim)[None, :]
        assert np.abs(np.cos(wrong) - c).max() > 1e-2


def test_rope_table_f64_closed_form():
    """Qwen3/Gemma2/ModernBERT tables (qwen3/mod.rs:131-153): angles in f64,
    stored f32, so each entry is the f64 closed form rounded once (half an f32
    ulp, plus libm's last-bit error in f64)."""
    for dim, theta, n in ((128, 1e6, 300), (256, 1e4, 64), (64, 160000.0, 100)):
        c, s = op.rope_table(dim, theta, n)
        i = np.arange(dim // 2)
        ang = np.arange(n, dtype=np.float64)[:, None] / np.power(theta, 2.0 * i / dim)[None, :]
        bound = np.maximum(np.abs(np.cos(ang)), np.abs(np.sin(ang))) * 2.0 ** -24 + 1e-15
        assert np.all(np.abs(c - np.cos(ang)) <= bound)
        assert np.all(np.abs(s - np.sin(ang)) <= bound)
        # position 1, frequency 0 is one radian
        assert c[1, 0] == np.float32(np.cos(1.0)) and s[1, 0] == np.float32(np.sin(1.0))
