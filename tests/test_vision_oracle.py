"""Pins oracle/exn_vision_oracle.py (the vision tower's CPU restatement): encode
against the reference's own inspect/ref_vision.py (vectors in
tests/golden/ref_vision_tiny.npz, written by make_ref_vision_vectors.py from the
same synthetic weights), and the pieces against closed forms, float64 brute force
and the index formulas of src/host.lisp:119-166."""
import math
import os

import numpy as np
import pytest

from oracle import exn_oracle as xo
from oracle import exn_vision_oracle as vo

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TINY = vo.VShape(width=144, heads=2, ffn=160, depth=4, deepstack=(1, 2, 3), out=96, side=6)


@pytest.fixture(scope="module")
def golden():
    return np.load(os.path.join(GOLDEN, "ref_vision_tiny.npz"))


@pytest.mark.parametrize("case", [0, 1, 2])
def test_encode_matches_reference_script(golden, case):
    """The whole tower at a narrow width (4 blocks, deepstack after 1, 2, 3) on a
    wide grid, a single merge block and a grid taller than the position table,
    against inspect/ref_vision.py run on the same weights: both float32 numpy."""
    seed, h, w = (int(v) for v in golden["c%d_meta" % case])
    wt = vo.SynthVision(seed, TINY)
    sums = np.array([float(np.sum(wt(n), dtype=np.float64)) for n, _ in vo.vision_expected(TINY)])
    assert np.array_equal(sums, golden["c%d_wsum" % case])          # the generator is unchanged
    px = golden["c%d_px" % case]
    assert np.array_equal(px, vo.synth_picture(seed + case, h, w))
    got = vo.encode(px, wt, TINY)
    for k in ("embed", "blk0", "merged"):
        assert got[k].shape == golden["c%d_%s" % (case, k)].shape
        assert xo.rel_l2(got[k], golden["c%d_%s" % (case, k)]) < 1e-6, k
    assert xo.rel_l2(np.stack(got["ds"]), golden["c%d_ds" % case]) < 1e-6
    # the deepstack mergers read different blocks' states
    ds = golden["c%d_ds" % case]
    assert xo.rel_l2(ds[0], ds[1]) > 0.05 and xo.rel_l2(ds[1], ds[2]) > 0.05


def test_merge_order_closed_form():
    """Patch k of a gh x gw grid: block (k // 4) in row-major order over the
    (gh/2) x (gw/2) blocks, then (k % 4) as (row, col) inside it."""
    gh, gw = 6, 10
    rows, cols = vo.merge_order(gh, gw)
    k = np.arange(gh * gw)
    blk, inner = k // 4, k % 4
    assert np.array_equal(rows, 2 * (blk // (gw // 2)) + inner // 2)
    assert np.array_equal(cols, 2 * (blk % (gw // 2)) + inner % 2)
    assert len(set(zip(rows.tolist(), cols.tolist()))) == gh * gw


def test_interp_taps_corners_and_identity():
    side = 7
    for size in (2, 5, 7, 12):
        idx = np.arange(size)
        taps, w = vo.interp_taps(idx, size, side)
        assert np.allclose(w.sum(1), 1.0, atol=1e-15)
        assert taps[0, 0] == 0 and w[0, 0] == 1.0                        # first index: the first entry
        last = (taps[-1] * (w[-1] > 0)).max()
        assert last == side - 1 and w[-1][taps[-1] == side - 1].sum() == 1.0
        src = idx * (side - 1) / (size - 1)                               # the interpolated coordinate
        assert np.allclose((taps * w).sum(1), src, atol=1e-12)
    taps, w = vo.interp_taps(np.arange(side), side, side)                 # same size: the table itself
    assert np.array_equal(taps[:, 0], np.arange(side)) and np.array_equal(w[:, 0], np.ones(side))


def test_pos_embed_is_the_table_when_the_grid_matches_it():
    side, d = 6, 8
    table = xo.normal(5, 77, side * side * d).reshape(side * side, d)
    rows, cols = vo.merge_order(side, side)
    pe = vo.pos_embed(table, rows, cols, side, side, side)
    assert np.array_equal(pe, table[rows * side + cols])


def test_pos_embed_against_float64_bilinear():
    side, d, gh, gw = 6, 4, 10, 4
    table = xo.normal(5, 78, side * side * d).reshape(side * side, d)
    rows, cols = vo.merge_order(gh, gw)
    pe = vo.pos_embed(table, rows, cols, gh, gw, side)
    t = table.astype(np.float64).reshape(side, side, d)
    for k in range(len(rows)):
        y, x = rows[k] * (side - 1) / (gh - 1), cols[k] * (side - 1) / (gw - 1)
        y0, x0 = min(int(y), side - 2), min(int(x), side - 2)
        fy, fx = y - y0, x - x0
        want = ((1 - fy) * (1 - fx) * t[y0, x0] + (1 - fy) * fx * t[y0, x0 + 1]
                + fy * (1 - fx) * t[y0 + 1, x0] + fy * fx * t[y0 + 1, x0 + 1])
        assert np.allclose(pe[k], want, atol=1e-5)


def test_rotary_angles_closed_form():
    """Dim j < 18 turns by the patch's row at 10000^(-j/18), 18 <= j < 36 by its
    column at 10000^(-(j-18)/18); dims 36..71 repeat them (src/host.lisp:154-166)."""
    rows, cols = vo.merge_order(8, 12)
    cos, sin = vo.rotary(rows, cols, 72)
    j = np.arange(36)
    inv = 10000.0 ** (-(j % 18) / 18.0)
    pos = np.where(j < 18, rows[:, None], cols[:, None])
    ang = pos * inv
    assert np.allclose(cos[:, :36], np.cos(ang), atol=2e-6) and np.allclose(sin[:, :36], np.sin(ang), atol=2e-6)
    assert np.array_equal(cos[:, 36:], cos[:, :36]) and np.array_equal(sin[:, 36:], sin[:, :36])


def test_rope_is_a_rotation_of_each_pair():
    """rotate_half pairs dim i with i + 36: each pair turns by its angle, so the
    norm of every (i, i + 36) pair is kept and q.k depends on the positions'
    difference only."""
    n, hd = 5, 72
    t = xo.normal(3, 79, n * 2 * hd).reshape(n, 2, hd)
    rows, cols = np.arange(n), np.arange(n)[::-1].copy()
    cos, sin = vo.rotary(rows, cols, hd)
    r = vo.rope(t, cos, sin)
    pair = lambda a: a[..., :36] ** 2 + a[..., 36:] ** 2
    assert np.allclose(pair(r), pair(t), rtol=1e-5)
    # the same vector at two positions shifted together: the dot product is unchanged
    q, k = t[0, 0], t[1, 0]
    rq = lambda v, pr, pc: vo.rope(np.broadcast_to(v, (1, 1, hd)).copy(), *vo.rotary(np.array([pr]), np.array([pc]), hd))[0, 0]
    assert abs(float(rq(q, 3, 5) @ rq(k, 1, 2)) - float(rq(q, 9, 11) @ rq(k, 7, 8))) < 1e-4


def test_attention_against_float64():
    n, heads, hd = 9, 2, 72
    q, k, v = (xo.normal(4, 80 + i, n * heads * hd).reshape(n, heads, hd) for i in range(3))
    got = vo.attention(q, k, v)
    for h in range(heads):
        s = q[:, h].astype(np.float64) @ k[:, h].astype(np.float64).T / math.sqrt(hd)
        p = np.exp(s - s.max(1, keepdims=True))
        want = (p / p.sum(1, keepdims=True)) @ v[:, h].astype(np.float64)
        assert np.allclose(got[:, h], want, atol=1e-5)


def test_gelus_and_layernorm_closed_forms():
    x = np.linspace(-6, 6, 97, dtype=np.float32)
    erf = np.array([math.erf(float(v) / math.sqrt(2)) for v in x])
    assert np.allclose(vo.gelu_erf(x), 0.5 * x * (1 + erf), atol=1e-6)
    t = np.tanh(math.sqrt(2 / math.pi) * (x.astype(np.float64) + 0.044715 * x.astype(np.float64) ** 3))
    assert np.allclose(vo.gelu_tanh(x), 0.5 * x * (1 + t), atol=1e-6)
    y = xo.normal(6, 81, 3 * 50).reshape(3, 50) * 3 + 2
    z = vo.layernorm(y, np.ones(50, np.float32), np.zeros(50, np.float32))
    assert np.allclose(z.mean(1), 0, atol=1e-6) and np.allclose(z.var(1), 1, atol=1e-4)


def test_schema():
    names = dict(vo.vision_expected())
    assert len(names) == 4 + 27 * 12 + 3 * 6 + 6
    assert names["v.blk.26.attn_qkv.weight"] == (3456, 1152)
    assert names["v.blk.0.ffn_up.weight"] == (4304, 1152) and names["v.blk.0.ffn_down.weight"] == (1152, 4304)
    assert names["v.deepstack.16.fc1.weight"] == (4608, 4608) and names["mm.2.weight"] == (4096, 4608)
    assert names["v.position_embd.weight"] == (2304, 1152)


def test_synthetic_matrices_are_fp16_and_vectors_are_not():
    wt = vo.SynthVision(2, TINY)
    a = wt("v.blk.1.attn_qkv.weight")
    assert np.array_equal(a.astype(np.float16).astype(np.float32), a)
    b = wt("v.blk.1.attn_qkv.bias")
    assert not np.array_equal(b.astype(np.float16).astype(np.float32), b)
    g = wt("v.blk.1.ln1.weight")
    assert abs(float(g.mean()) - 1) < 0.05
