"""The prompt encoder (Qwen3-VL-8B's text model) on the GPU through the C ABI, against the
oracle (oracle/exn_encoder_oracle.py; parity unpinned against illatio, whose arithmetic the
reference does not vendor).  The products take bf16 activations and the Q8_0 weights
dequantised to bf16, attention fp16 operands, as the DiT's blocks do.  Through the text
model's attention (no gates: every block's output is the residual's bulk) that rounding
leaves the states about 1% from the fp32 oracle after 2 blocks and 2.3% after 36, and an
oracle that rounds at the same points lands as far: the bar is relative L2 1.5e-2 for 2
blocks, 3e-2 for all 36, with the rounding model checked beside it.  Needs an MI355X."""
import sys

import numpy as np
import pytest

import exn_hip as X
from oracle import exn_encoder_oracle as eo
from oracle import exn_oracle as xo

pytestmark = pytest.mark.gpu
SEED = 31
VOCAB = 8192


def say(*a):
    print("[gpu]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    c = X.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def enc2(ctx):
    say("encoder synth, 2 layers")
    e = X.load_encoder(seed=SEED, layers=2, vocab=VOCAB, ctx=ctx)
    yield e
    e.destroy()


@pytest.fixture(scope="module")
def owt2():
    return eo.SynthEncoder(SEED, eo.EShape(layers=2))


# 1, 37: the few-row 128 x 256 tiles; 200: 256 x 128 (ragged rows, q | k | v split 5 ways); 1025 on:
# past the split-K path
@pytest.mark.parametrize("n", [1, 37, 200, 300, 1024, 1025, 1100])
def test_states_two_layers_against_oracle(enc2, owt2, n):
    say("encoder states, 2 layers, n", n)
    ids = eo.synth_ids(SEED + n, n, VOCAB)
    got = X.encoder_states(enc2, ids)
    want = eo.states(owt2, ids, s=eo.EShape(layers=2))
    err = xo.rel_l2(got, want)
    say("rel l2", err)
    assert err < 1.5e-2
    assert np.isfinite(got).all()


def test_states_of_an_edit_prompt(enc2, owt2):
    """5 text tokens, a 4 x 6 picture's rows (merged, and deepstack added after layers 0 and
    1), 9 more: positions and picture rows as encode-edit-prompt gives them."""
    a0, gh, gw, after = 5, 4, 6, 9
    pos = eo.edit_positions(a0, gh, gw, after)
    n = len(pos)
    ids = eo.synth_ids(SEED + 1, n, VOCAB)
    merged, deep = eo.synth_picture_rows(SEED + 2, gh * gw)
    got = X.encoder_states(enc2, ids, pos, (a0, merged, deep))
    want = eo.states(owt2, ids, pos, (a0, merged, deep), s=eo.EShape(layers=2))
    err = xo.rel_l2(got, want)
    say("edit rel l2", err)
    assert err < 1.5e-2
    plain = X.encoder_states(enc2, ids)
    assert xo.rel_l2(plain[a0 + gh * gw:], got[a0 + gh * gw:]) > 1e-2     # the picture is seen after it


def test_set_from_gguf_records_equals_synth(ctx, enc2, owt2):
    """exn_enc_set with block_q8_0 records and F32 norms (the file's kinds) gives the synthetic
    model's states bit for bit."""
    e = X.Encoder(ctx, 2)
    try:
        qs, d = owt2.q8("token_embd.weight")
        e.set("token_embd.weight", X.Q8_0, xo.q8_0_to_blocks(qs, d), 4096, VOCAB)
        for name, shape in eo.enc_expected(eo.EShape(layers=2))[1:]:
            if len(shape) == 1:
                e.set(name, X.F32, owt2(name), shape[0], 1)
            else:
                e.set(name, X.Q8_0, xo.q8_0_to_blocks(*owt2.q8(name)), shape[1], shape[0])
        e.set("output_norm.weight", X.F32, np.ones(4096, np.float32), 4096, 1)
        e.check()
        ids = eo.synth_ids(SEED + 3, 50, VOCAB)
        assert np.array_equal(X.encoder_states(e, ids), X.encoder_states(enc2, ids))
    finally:
        e.destroy()


def test_states_full_depth(ctx):
    """All 36 blocks on 48 tokens against the oracle (its layers made as read); then what the
    encoder's distance does downstream: the DiT (2 blocks, an 8 x 8 latent) on the GPU's states
    against the oracle's DiT on the oracle's states -- the whole prompt-to-velocity chain within
    the DiT's per-block bar (relative L2 <= 1e-2), the GPU DiT on the oracle's states beside it."""
    say("encoder synth, 36 layers")
    e = X.load_encoder(seed=SEED, layers=36, vocab=VOCAB, ctx=ctx)
    try:
        ids = eo.synth_ids(SEED + 4, 48, VOCAB)
        got = X.encoder_states(e, ids)
        w, s = e.memory()
        assert w > 8e9
    finally:
        e.destroy()
    want = eo.states(eo.SynthEncoder(SEED, eo.EShape(), keep=False), ids)
    err = xo.rel_l2(got, want)
    say("36 layers rel l2", err)
    assert err < 3e-2 and np.isfinite(got).all()
    dseed, hh, ww, sigma = 9, 8, 8, 0.95418
    d = X.Dit(ctx, 2)
    try:
        d.synth(dseed)
        d.check()
        lat = xo.synth_inputs(dseed, 1, hh, ww)[1]
        p = got.shape[0]
        v_chain = X.dit_velocity(d, np.ascontiguousarray(got, np.float32), p, lat, hh, ww, sigma)
        v_dit = X.dit_velocity(d, np.ascontiguousarray(want, np.float32), p, lat, hh, ww, sigma)
    finally:
        d.destroy()
    ref = xo.forward(xo.SynthWeights(dseed), want.astype(np.float32), lat, sigma, layers=2)
    e_chain, e_dit = xo.rel_l2(v_chain, ref), xo.rel_l2(v_dit, ref)
    say("DiT velocity from the GPU encoder's states rel-L2 %.2e (from the oracle's states %.2e)" % (e_chain, e_dit))
    assert e_chain < 1e-2 and e_dit < 1e-2


def test_the_distance_is_the_rounding(enc2, owt2):
    """The oracle with bf16 matrices and product inputs and fp16 q, k, v (the GPU's rounding
    points) is as far from the fp32 oracle as the GPU is, and nearer the GPU than that."""
    ids = eo.synth_ids(SEED + 5, 64, VOCAB)
    got = X.encoder_states(enc2, ids)
    exact = eo.states(owt2, ids, s=eo.EShape(layers=2))
    model = eo.states(owt2, ids, s=eo.EShape(layers=2), bf16=True)
    g, m, gm = xo.rel_l2(got, exact), xo.rel_l2(model, exact), xo.rel_l2(got, model)
    say("gpu-fp32", g, "model-fp32", m, "gpu-model", gm)
    assert abs(g - m) < 0.25 * g and gm < g


@pytest.mark.parametrize("n", [40, 300, 1100])   # the split-K path (5 and 2 splits) and whole tiles
def test_resident_expansion_equals_q8_products(enc2, n):
    """The products from the resident bf16 expansions (the default) and from Q8_0 dequantised
    in the pipeline take the same operand values in the same order: the states bit for bit."""
    ids = eo.synth_ids(SEED + 6 + n, n, VOCAB)
    a = X.encoder_states(enc2, ids)
    enc2.resident(False)
    try:
        b = X.encoder_states(enc2, ids)
    finally:
        enc2.resident(True)
    assert np.array_equal(a, b)


def test_a_set_matrix_remakes_its_expansion(ctx, owt2):
    """A matrix set after its expansion was made is multiplied from the new values; the
    expansions are made by the first prompt longer than 256 tokens, not by shorter ones."""
    e = X.load_encoder(seed=SEED, layers=2, vocab=VOCAB, ctx=ctx)
    try:
        w0, _ = e.memory()
        X.encoder_states(e, eo.synth_ids(SEED + 8, 40, VOCAB))
        assert e.memory()[0] == w0                            # a short prompt leaves them unmade
        ids = eo.synth_ids(SEED + 7, 300, VOCAB)
        before = X.encoder_states(e, ids)
        assert e.memory()[0] > w0
        other = eo.SynthEncoder(SEED + 100, eo.EShape(layers=2))
        name = "blk.1.ffn_down.weight"
        shape = dict(eo.enc_expected(eo.EShape(layers=2)))[name]
        e.set(name, X.Q8_0, xo.q8_0_to_blocks(*other.q8(name)), shape[1], shape[0])
        after = X.encoder_states(e, ids)
        e.resident(False)
        q8 = X.encoder_states(e, ids)
        assert np.array_equal(after, q8) and not np.array_equal(after, before)
    finally:
        e.destroy()


def test_release_frees_scratch_and_keeps_weights(enc2):
    """encoder release (the scratch freed, weights and expansions kept): the memory it reports
    drops to the weights, and the next prompt makes its buffers again (no larger than before)
    with the same states."""
    ids = eo.synth_ids(SEED + 9, 37, VOCAB)
    a = X.encoder_states(enc2, ids)
    w, s = enc2.memory()
    assert s > 0
    enc2.release()
    assert enc2.memory() == (w, 0)
    b = X.encoder_states(enc2, ids)
    assert np.array_equal(a, b) and 0 < enc2.memory()[1] <= s


def test_encoder_errors(ctx, enc2):
    e = X.Encoder(ctx, 2)
    try:
        with pytest.raises(X.ExnError) as ex:
            e.check()
        assert ex.value.code == X.ESTATE
        with pytest.raises(X.ExnError) as ex:
            e.set("blk.2.attn_norm.weight", X.F32, np.ones(4096, np.float32), 4096, 1)
        assert ex.value.code == X.EINVAL                      # past the layers
        with pytest.raises(X.ExnError) as ex:
            e.set("blk.0.attn_k.weight", X.Q8_0, np.zeros(4096 * 34 * 32, np.uint8), 4096, 4096)
        assert ex.value.code == X.EINVAL                      # k has 1024 rows
    finally:
        e.destroy()
    with pytest.raises(X.ExnError) as ex:
        X.encoder_states(enc2, np.array([0, VOCAB], np.int32))
    assert ex.value.code == X.EINVAL
