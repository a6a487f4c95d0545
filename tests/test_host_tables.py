"""The library's host-side tables against the oracle, without a GPU: the
positions every sequence row gets (dit-positions, src/host.lisp:37-50; integer
work, bit-exact) and the cos/sin table the step uploads (rope-table,
src/host.lisp:19-30; within one float32 ulp), through the C ABI test hook
exn_dit_rope_table, for odd image sizes and for edit layouts with rh != rw."""
import numpy as np
import pytest

import exn_hip as X
from oracle import exn_oracle as xo

# (text rows p, image h, w, reference picture (a, rh, rw) or None)
CASES = [
    (0, 1, 1, None), (1, 3, 5, None), (7, 5, 3, None), (256, 64, 64, None), (256, 96, 64, None), (33, 17, 9, None),
    (12, 3, 4, (2, 2, 3)), (9, 5, 7, (0, 3, 6)), (20, 7, 4, (20, 5, 2)), (512, 64, 64, (8, 64, 64)),
    (31, 9, 11, (13, 7, 3)),
]


def ulps(a, b):
    """Distance in float32 units in the last place (same-sign values, zeros equal)."""
    ia = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    ib = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return np.abs(ia - ib)


@pytest.mark.parametrize("p,h,w,ref", CASES)
def test_positions_and_rope_table_match_the_oracle(p, h, w, ref):
    pos, cs = X.rope_table(p, h, w, ref)
    nref = 0 if ref is None else ref[1] * ref[2]
    want_pos = xo.positions(p + nref, h, w, ref)
    assert pos.shape == want_pos.shape
    assert (pos == want_pos.astype(np.int64)).all()
    cos, sin = xo.rope_tables(want_pos)
    assert ulps(cs[:, 0::2], cos).max() <= 1 and ulps(cs[:, 1::2], sin).max() <= 1


def test_rope_table_against_the_angles_in_double():
    """Each pair's angle from its axis and index alone: pos_a / 10000^(2i/d_a), axes (16, 56, 56)."""
    pos, cs = X.rope_table(5, 3, 7, (2, 2, 2))
    j = 0
    for a, d in enumerate((16, 56, 56)):
        for i in range(d // 2):
            ang = pos[:, a].astype(np.float64) / 10000.0 ** (2 * i / d)
            assert ulps(cs[:, 2 * j], np.cos(ang).astype(np.float32)).max() <= 1
            assert ulps(cs[:, 2 * j + 1], np.sin(ang).astype(np.float32)).max() <= 1
            j += 1
    assert j == 64


def test_rope_table_refuses_bad_layouts():
    with pytest.raises(X.ExnError) as e:
        X.call("exn_dit_rope_table", 4, 2, 2, 1, 5, 2, 2, 100, None, None)   # a past the text
    assert e.value.code == X.EINVAL
    with pytest.raises(X.ExnError) as e:
        X.call("exn_dit_rope_table", 4, 2, 2, 0, 0, 0, 0, 7, None, None)     # 8 rows, room for 7
    assert e.value.code == X.EINVAL
    X.call("exn_dit_rope_table", 4, 2, 2, 0, 0, 0, 0, 8, None, None)


# --- the prompt encoder's M-RoPE table (mrope-table, src/encoder.lisp:26-39) ----------------

@pytest.mark.parametrize("case", ["text", "edit"])
def test_encoder_rope_table_matches_the_oracle(case):
    """exn_enc_rope_table against the oracle's mrope_tables: text positions 0 .. 299, and an edit
    prompt's positions (5 text tokens, a 7 x 11 picture, 9 more), within one float32 ulp
    (angles above 2^12 radians are not reached here)."""
    from oracle import exn_encoder_oracle as eo
    pos = eo.text_positions(300) if case == "text" else eo.edit_positions(5, 7, 11, 9)
    cs = X.enc_rope_table(len(pos), None if case == "text" else pos)
    cos, sin = eo.mrope_tables(pos)
    assert ulps(cs[:, 0::2], cos).max() <= 1 and ulps(cs[:, 1::2], sin).max() <= 1
