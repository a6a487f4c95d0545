"""Pins oracle/exn_encoder_oracle.py (the prompt encoder's text model).  Its arithmetic
lives in illatio, which the reference does not vendor, so no vector of the reference's
covers it (parity unpinned against illatio's own arithmetic).  These checks hold it to the
published model -- transformers' Qwen3VLTextModel with the same weights -- and to what the
mathematics and the reference's own text fix: M-RoPE on text positions is 1-D RoPE with
theta 5e6 (docs/design.md:46-48), the sections are 24/20/20, attention is causal,
grouped key/value heads equal repeated ones, rotate_half is a rotation, and the
picture's rows enter where call-with-picture-rows puts them (src/encoder.lisp:69-110)."""
import math

import numpy as np
import pytest

from oracle import exn_encoder_oracle as eo
from oracle import exn_oracle as xo

SMALL = eo.EShape(width=512, layers=2, heads=4, kv_heads=2, head_dim=128, ffn=512, vocab=512)


@pytest.fixture(scope="module")
def wt():
    return eo.SynthEncoder(5, SMALL)


def test_mrope_on_text_positions_is_1d_rope():
    pos = eo.text_positions(300)
    cos, sin = eo.mrope_tables(pos)
    i, j = np.arange(300)[:, None].astype(np.float64), np.arange(64)[None, :]
    ang = i * 5e6 ** (-(2.0 * j) / 128.0)
    assert np.allclose(cos, np.cos(ang), atol=1e-6) and np.allclose(sin, np.sin(ang), atol=1e-6)


def test_mrope_sections_are_24_20_20():
    """A picture token at (t, h, w) = (3, 11, 29): 24 frequencies turn by t, 20 by h, 20 by w."""
    pos = np.array([[3, 11, 29]])
    cos, sin = eo.mrope_tables(pos)
    inv = 5e6 ** (-(2.0 * np.arange(64)) / 128.0)
    cand = np.array([3, 11, 29], np.float64)[:, None] * inv            # (3, 64)
    dist = np.abs(cos[0] - np.cos(cand)) + np.abs(sin[0] - np.sin(cand))
    which = dist.argmin(0)                                              # the axis each frequency turns by
    assert np.sort(dist, 0)[1].min() > 10 * dist.min(0).max()           # every frequency tells them apart
    assert np.bincount(which, minlength=3).tolist() == [24, 20, 20]


def test_edit_positions_follow_the_picture():
    pos = eo.edit_positions(5, 3, 4, 6)
    assert pos.shape == (5 + 12 + 6, 3)
    assert (pos[:5] == np.arange(5)[:, None]).all()
    assert (pos[5:17, 0] == 5).all() and pos[5 + 4 * 2 + 3].tolist() == [5, 7, 8]
    assert pos[17].tolist() == [9, 9, 9] and pos[-1].tolist() == [14, 14, 14]   # 5 + max(3, 4) on


def test_rope_half_is_a_rotation_and_relative():
    x = xo.normal(1, 9001, 2 * 3 * 128).reshape(2, 3, 128)
    cos, sin = eo.mrope_tables(eo.text_positions(2, 17))
    r = eo.rope_half(x, cos, sin)
    pair = lambda a: a[..., :64] ** 2 + a[..., 64:] ** 2
    assert np.allclose(pair(r), pair(x), rtol=1e-5)
    q, k = x[0, 0], x[1, 0]
    at = lambda v, p: eo.rope_half(v[None, None], *eo.mrope_tables(eo.text_positions(1, p)))[0, 0]
    assert abs(float(at(q, 40) @ at(k, 33)) - float(at(q, 107) @ at(k, 100))) < 1e-3


def test_rmsnorm_closed_form():
    x = xo.normal(2, 9002, 4 * 64).reshape(4, 64) * np.float32(3)
    y = eo.rmsnorm(x, np.ones(64, np.float32))
    assert np.allclose((y.astype(np.float64) ** 2).mean(-1), 1.0, atol=1e-5)


def test_causal(wt):
    ids = eo.synth_ids(3, 24, SMALL.vocab)
    full = eo.states(wt, ids, s=SMALL)
    head = eo.states(wt, ids[:15], s=SMALL)
    assert np.allclose(full[:15], head, atol=2e-5 * np.abs(head).max())
    assert xo.rel_l2(eo.states(wt, ids[1:], s=SMALL)[14:], full[15:]) > 1e-3     # the prefix matters


def test_grouped_heads_equal_repeated_heads(wt):
    """Query head h reads key/value head h // 2 (transformers' repeat_kv): the same model with
    every key/value head written out twice in a row (kv_heads = heads) gives the same states."""
    rep = eo.EShape(width=512, layers=2, heads=4, kv_heads=4, head_dim=128, ffn=512, vocab=512)

    class Repeated:
        def __call__(self, name):
            a = wt(name)
            if name.endswith("attn_k.weight") or name.endswith("attn_v.weight"):
                a = np.repeat(a.reshape(SMALL.kv_heads, 128, -1), 2, axis=0).reshape(-1, a.shape[1])
            return a

    ids = eo.synth_ids(4, 17, SMALL.vocab)
    assert np.allclose(eo.states(Repeated(), ids, s=rep), eo.states(wt, ids, s=SMALL), atol=1e-5)


def test_picture_rows_enter_as_call_with_picture_rows(wt):
    ids = eo.synth_ids(5, 20, SMALL.vocab)
    emb = wt("token_embd.weight")[ids[6:10]]
    zero = np.zeros((3, 4, SMALL.width), np.float32)
    plain = eo.states(wt, ids, s=SMALL)
    assert np.array_equal(eo.states(wt, ids, picture=(6, emb, zero), s=SMALL), plain)
    one = eo.EShape(width=512, layers=1, heads=4, kv_heads=2, head_dim=128, ffn=512, vocab=512)
    base = eo.states(wt, ids, s=one)
    delta = np.zeros_like(zero)
    delta[0] = xo.normal(6, 9003, 4 * SMALL.width).reshape(4, SMALL.width)
    got = eo.states(wt, ids, picture=(6, emb, delta), s=one)
    assert np.array_equal(got[:6], base[:6]) and np.array_equal(got[10:], base[10:])
    assert np.allclose(got[6:10], base[6:10] + delta[0], atol=1e-6)


def test_states_match_transformers_qwen3vl_text_model(wt):
    """The published model itself: transformers' Qwen3VLTextModel (the implementation the oracle
    restates; an installed library, not the reference) with the oracle's weights copied in and
    its final norm taken out, on an edit prompt's positions (t, h, w) with picture rows and two
    deepstack sets: the same states within float32 rounding."""
    torch = pytest.importorskip("torch")
    pytest.importorskip("transformers")
    from transformers import Qwen3VLTextConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextModel

    s = SMALL
    cfg = Qwen3VLTextConfig(vocab_size=s.vocab, hidden_size=s.width, intermediate_size=s.ffn,
                            num_hidden_layers=s.layers, num_attention_heads=s.heads, num_key_value_heads=s.kv_heads,
                            head_dim=s.head_dim, rms_norm_eps=1e-6, max_position_embeddings=4096,
                            rope_parameters={"rope_type": "default", "rope_theta": eo.ROPE_BASE,
                                             "mrope_section": [24, 20, 20], "mrope_interleaved": True})
    cfg._attn_implementation = "eager"
    torch.manual_seed(0)
    model = Qwen3VLTextModel(cfg).eval()
    model.norm = torch.nn.Identity()                      # the states before the final norm
    names = {"self_attn.q_proj": "attn_q", "self_attn.k_proj": "attn_k", "self_attn.v_proj": "attn_v",
             "self_attn.o_proj": "attn_output", "self_attn.q_norm": "attn_q_norm", "self_attn.k_norm": "attn_k_norm",
             "input_layernorm": "attn_norm", "post_attention_layernorm": "ffn_norm", "mlp.gate_proj": "ffn_gate",
             "mlp.up_proj": "ffn_up", "mlp.down_proj": "ffn_down"}
    sd = {"embed_tokens.weight": torch.from_numpy(wt("token_embd.weight").copy())}
    for i in range(s.layers):
        for theirs, ours in names.items():
            sd["layers.%d.%s.weight" % (i, theirs)] = torch.from_numpy(wt("blk.%d.%s.weight" % (i, ours)).copy())
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected and all("rotary" in k or k.startswith("norm") for k in missing), (missing, unexpected)

    a0, gh, gw, after = 3, 2, 3, 4
    pos = eo.edit_positions(a0, gh, gw, after)
    n = len(pos)
    ids = eo.synth_ids(8, n, s.vocab)
    merged, deep = eo.synth_picture_rows(9, gh * gw, s.width)
    deep = deep[:2]                                        # two sets: after layers 0 and 1
    want = eo.states(wt, ids, pos, (a0, merged, deep), s=s)

    emb = torch.from_numpy(wt("token_embd.weight")[ids].copy())[None]
    emb[0, a0:a0 + gh * gw] = torch.from_numpy(merged)
    mask = torch.zeros(1, n, dtype=torch.bool)
    mask[0, a0:a0 + gh * gw] = True
    with torch.no_grad():
        out = model(inputs_embeds=emb, position_ids=torch.from_numpy(pos.T.copy())[:, None, :],
                    visual_pos_masks=mask, deepstack_visual_embeds=[torch.from_numpy(d) for d in deep],
                    use_cache=False).last_hidden_state[0].numpy()
    assert xo.rel_l2(want, out) < 2e-6
    # and a mistake the oracle could make shows: the h and w axes swapped in the table
    swapped = pos[:, [0, 2, 1]]
    assert xo.rel_l2(eo.states(wt, ids, swapped, (a0, merged, deep), s=s), out) > 1e-4
