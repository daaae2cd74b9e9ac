"""Whole-model parity on the MI355X through the C ABI: the encode-side pass
(GEMM/prefill shapes) and the decode-side pass (GEMV/step shapes) return the
oracle's distributions bit for bit, encode writes the oracle's bytes, decode
recovers the tokens."""
import concurrent.futures
import dataclasses

import numpy as np
import pytest

from tsac_hip.synthetic import WIDE, Geometry, bf16_float, pattern_tokens, random_model, random_tokens

pytestmark = pytest.mark.gpu

SMALL = Geometry(width=256, heads=2, head_width=128, ffn=512, temporal_layers=2, codebook_layers=1,
                 latent=256)
TINY = Geometry(width=256, heads=2, head_width=128, ffn=256, temporal_layers=1, codebook_layers=1,
                latent=256)


@pytest.fixture(scope="module")
def native():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    from tsac_hip import native

    native.library()
    return native


@pytest.fixture(scope="module")
def small(native):
    model = random_model(SMALL, seed=3)
    return model, native.HipModel(model)


@pytest.fixture(scope="module")
def reference_model(native):
    model = random_model(seed=1)
    return model, native.HipModel(model)


def _both_passes(native, hip_model, h, tokens):
    session = hip_model.session()
    encode = session.distributions(h, tokens, native.PASS_ENCODE)
    decode = session.distributions(h, tokens, native.PASS_DECODE)
    return encode, decode


@pytest.mark.parametrize("frames,batch,groups,books", [(17, 3, 1, 12), (35, 3, 2, 12), (17, 8, 16, 12),
                                                       (3, 8, 2, 12), (5, 3, 1, 7), (17, 1, 1, 12)])
def test_small_model_passes_match_oracle(native, oracle, small, frames, batch, groups, books):
    model, hip_model = small
    h = native.header(frames, batch, groups, books)
    tokens = pattern_tokens(frames * groups * books)
    encode, decode = _both_passes(native, hip_model, h, tokens)
    from oracle import header

    expected = oracle.model(model).distributions(header(frames, batch, groups, books), tokens, threads=4)
    assert np.array_equal(encode, decode), "encode-side and decode-side passes differ"
    assert np.array_equal(encode, expected)


@pytest.mark.parametrize("frames,batch,groups", [(17, 3, 1), (101, 3, 1), (35, 3, 2), (3, 8, 2)])
def test_stream_bytes_and_round_trip(native, oracle, small, frames, batch, groups):
    """GPU encode == oracle pack_normal bytes; GPU decode recovers the tokens."""
    model, hip_model = small
    h = native.header(frames, batch, groups, 12)
    tokens = random_tokens(frames, groups, 12, seed=frames)
    session = hip_model.session()
    stream = session.encode(h, tokens)
    from oracle import header

    assert stream == oracle.model(model).pack_normal(header(frames, batch, groups, 12), tokens, threads=4)
    assert np.array_equal(session.decode(stream), tokens)


def _recorder():
    before, after = [], []

    def on_before(p):
        before.append((p.frame, p.group, p.codebook, p.lane, p.step, p.token_offset))

    def on_after(p, bits):
        after.append((p.frame, p.group, p.codebook, p.lane, p.step, p.token_offset, bits))

    return before, after, on_before, on_after


@pytest.mark.parametrize("frames,batch,groups", [(35, 3, 2), (17, 8, 1)])
def test_observer_sees_the_oracle_positions_and_bits(native, oracle, small, frames, batch, groups):
    """EntropyObserver across the C ABI: encode reports every symbol in stream
    order with the bits the range coder spent on it, as the oracle's
    pack_normal (pinned to the reference's own) does; decode reports the same
    positions with 0 bits."""
    from oracle import header

    model, hip_model = small
    h = native.header(frames, batch, groups, 12)
    tokens = random_tokens(frames, groups, 12, seed=frames + groups)
    expected_stream, bits, positions = oracle.model(model).pack_normal_observed(header(frames, batch, groups, 12),
                                                                                 tokens, threads=3)
    with hip_model.session() as session:
        before, after, on_before, on_after = _recorder()
        stream = session.encode_observed(h, tokens, on_before, on_after)
        assert stream == expected_stream
        assert np.array_equal(np.array(before, np.uint64), positions)
        assert np.array_equal(np.array(after, np.uint64)[:, :6], positions)
        assert np.array_equal(np.array(after, np.uint64)[:, 6], bits)
        before, after, on_before, on_after = _recorder()
        assert np.array_equal(session.decode_observed(stream, on_before, on_after), tokens)
        assert np.array_equal(np.array(before, np.uint64), positions)
        assert np.array_equal(np.array(after, np.uint64)[:, :6], positions)
        assert not np.array(after, np.uint64)[:, 6].any()


def test_observer_can_stop_a_call_and_the_session_recovers(native, small):
    _, hip_model = small
    h = native.header(9, 3, 1, 12)
    tokens = pattern_tokens(9 * 12)
    with hip_model.session() as session:
        seen = []
        with pytest.raises(native.HipError, match="stopped by the observer"):
            session.encode_observed(h, tokens, after=lambda p, bits: seen.append(bits) or len(seen) == 5)
        assert len(seen) == 5
        stream = session.encode(h, tokens)
        with pytest.raises(native.HipError, match="stopped by the observer"):
            session.decode_observed(stream, before=lambda p: p.step == 2)
        assert np.array_equal(session.decode_observed(stream), tokens)


def test_rollover_replay(native, oracle):
    """1026 frames in one lane: context reset with the 256-frame replay."""
    model = random_model(TINY, seed=5)
    hip_model = native.HipModel(model)
    h = native.header(1026, 1, 1, 1)
    tokens = pattern_tokens(1026)
    session = hip_model.session()
    stream = session.encode(h, tokens)
    from oracle import header

    assert stream == oracle.model(model).pack_normal(header(1026, 1, 1, 1), tokens)
    assert np.array_equal(session.decode(stream), tokens)
    encode, decode = _both_passes(native, hip_model, h, tokens)
    assert np.array_equal(encode, decode)


def test_reference_geometry(native, oracle, reference_model):
    """Full reference geometry: 12 + 3 layers, width 512, 4 x 128 heads."""
    model, hip_model = reference_model
    h = native.header(6, 3, 1, 12)
    tokens = random_tokens(6, 1, 12, seed=9)
    encode, decode = _both_passes(native, hip_model, h, tokens)
    from oracle import header

    oh = header(6, 3, 1, 12)
    expected = oracle.model(model).distributions(oh, tokens, threads=3)
    assert np.array_equal(encode, decode)
    assert np.array_equal(encode, expected)
    assert np.all(np.isfinite(bf16_float(encode)))
    session = hip_model.session()
    stream = session.encode(h, tokens)
    assert stream == oracle.model(model).pack_normal(oh, tokens, threads=3)
    assert np.array_equal(session.decode(stream), tokens)


@pytest.mark.parametrize("frames,batch", [(5, 1), (4, 2), (8, 8)])
def test_reference_geometry_lane_counts(native, oracle, reference_model, frames, batch):
    """The decode step's workgroup layouts at 1, 2 and 8 lanes (with 8 lanes
    the codebook attention runs inside the out projection but the layer sets
    are not paired; with 1 and 2 lanes both apply)."""
    model, hip_model = reference_model
    h = native.header(frames, batch, 1, 12)
    tokens = random_tokens(frames, 1, 12, seed=frames + batch)
    encode, decode = _both_passes(native, hip_model, h, tokens)
    from oracle import header

    oh = header(frames, batch, 1, 12)
    expected = oracle.model(model).distributions(oh, tokens, threads=4)
    assert np.array_equal(encode, decode)
    assert np.array_equal(encode, expected)
    session = hip_model.session()
    stream = session.encode(h, tokens)
    assert stream == oracle.model(model).pack_normal(oh, tokens, threads=4)
    assert np.array_equal(session.decode(stream), tokens)


@pytest.fixture(scope="module")
def wide_model(native):
    model = random_model(WIDE, seed=2)
    hip_model = native.HipModel(model)
    yield model, hip_model
    hip_model.close()


@pytest.mark.parametrize("frames,batch", [(2, 2), (3, 1), (8, 8)])
def test_wide_geometry(native, oracle, wide_model, frames, batch):
    """Width 1024, FFN 4096, 16 x 64 heads: two codebook heads per wave in the
    out tiles, which run on the attention workgroups; with 8 lanes the groups
    are scaled down and each of those workgroups takes several tiles."""
    model, hip_model = wide_model
    h = native.header(frames, batch, 1, 12)
    tokens = random_tokens(frames, 1, 12, seed=4 + batch)
    encode, decode = _both_passes(native, hip_model, h, tokens)
    from oracle import header

    expected = oracle.model(model).distributions(header(frames, batch, 1, 12), tokens, threads=4)
    assert np.array_equal(encode, decode)
    assert np.array_equal(encode, expected)


def test_wide_geometry_long_context(native, wide_model):
    """Contexts past 512 frames at width 1024: every wave of a temporal query
    then takes a second block of keys, requested into LDS at the job's start;
    1030 frames also cross the 1024-frame rollover. The decode pass (frame
    steps) equals the encode pass (batched known tokens) bit for bit, and the
    stream decodes back to its tokens."""
    _, hip_model = wide_model
    h = native.header(1030, 1, 1, 12)
    tokens = random_tokens(1030, 1, 12, seed=11)
    encode, decode = _both_passes(native, hip_model, h, tokens)
    assert np.array_equal(encode, decode)
    session = hip_model.session()
    assert np.array_equal(session.decode(session.encode(h, tokens)), tokens)


def test_run_to_run_determinism(native, small):
    _, hip_model = small
    h = native.header(40, 3, 1, 12)
    tokens = random_tokens(40, 1, 12, seed=1)
    a, b = hip_model.session(), hip_model.session()
    assert a.encode(h, tokens) == b.encode(h, tokens) == a.encode(h, tokens)
    d1 = a.distributions(h, tokens, native.PASS_ENCODE)
    assert np.array_equal(d1, b.distributions(h, tokens, native.PASS_ENCODE))


def test_decode_rejects_corruption_and_session_recovers(native, small):
    _, hip_model = small
    h = native.header(9, 3, 1, 12)
    tokens = pattern_tokens(9 * 12)
    session = hip_model.session()
    stream = bytearray(session.encode(h, tokens))
    bad = bytearray(stream)
    bad[-1] ^= 1
    with pytest.raises(native.HipError, match="CRC"):
        session.decode(bytes(bad))
    bad = bytearray(stream)
    bad[14] = 0xFF  # initial interval byte (tests/metal_optimized.cpp:607-630)
    bad[15] = 0xFF
    bad[16] = 0xFF
    with pytest.raises(native.HipError):
        session.decode(bytes(bad))
    assert np.array_equal(session.decode(bytes(stream)), tokens)
    session.clear()
    assert np.array_equal(session.decode(bytes(stream)), tokens)


def test_encode_validates_inputs(native, small):
    _, hip_model = small
    session = hip_model.session()
    with pytest.raises(native.HipError, match="token count"):
        session.encode(native.header(3, 1, 1, 12), np.zeros(5, np.uint16))
    with pytest.raises(native.HipError, match="alphabet"):
        session.encode(native.header(1, 1, 1, 1), np.array([1024], np.uint16))
    with pytest.raises(native.HipError, match="codebook"):
        session.encode(native.header(1, 1, 1, 13), np.zeros(13, np.uint16))


@pytest.mark.parametrize("geometry", ["small", "reference"])
def test_concurrent_sessions_on_two_threads(native, small, reference_model, geometry):
    """Two sessions of one model driven from two host threads at once give the
    streams and tokens one session gives alone (tests/audio_analyzer.cpp:109-186);
    the reference geometry runs the persistent frame-step launch in both."""
    model, hip_model = small if geometry == "small" else reference_model
    frames = 40 if geometry == "small" else 24
    h = native.header(frames, 3, 1, 12)
    tokens = [random_tokens(frames, 1, 12, seed=40 + i) for i in range(2)]
    with hip_model.session() as alone:
        expected = [alone.encode(h, t) for t in tokens]

    def work(i):
        with hip_model.session() as session:
            out = []
            for _ in range(3):
                stream = session.encode(h, tokens[i])
                out.append((stream, session.decode(stream)))
            return out

    with concurrent.futures.ThreadPoolExecutor(2) as pool:
        results = list(pool.map(work, range(2)))
    for i, runs in enumerate(results):
        for stream, decoded in runs:
            assert stream == expected[i]
            assert np.array_equal(decoded, tokens[i])


def test_nonfinite_activation_is_an_error_and_the_session_recovers(native, reference_model):
    """A feedback embedding row of +inf (BF16 0x7f80) reaches the activations
    only when its symbol is coded: every pass that meets it fails with the
    nonfinite-activation error (tests/metal_range.cpp:21-61), in the frame-step
    launch too, and the same session then codes a stream that avoids it."""
    model, clean = reference_model
    poisoned = dataclasses.replace(model, embeddings=model.embeddings.copy())
    poisoned.embeddings[0, 1023, :] = 0x7F80
    frames, batch = 6, 3
    h = native.header(frames, batch, 1, 12)
    bad = random_tokens(frames, 1, 12, seed=12) % 1023
    bad[2 * 12 + 0] = 1023  # frame 2 (lane 1, step 0), book 0
    good = random_tokens(frames, 1, 12, seed=13) % 1023
    with clean.session() as session:
        bad_stream = session.encode(h, bad)
        good_stream = session.encode(h, good)
    with native.HipModel(poisoned) as hip_poisoned, hip_poisoned.session() as session:
        for call in (lambda: session.encode(h, bad), lambda: session.decode(bad_stream),
                     lambda: session.distributions(h, bad, native.PASS_ENCODE),
                     lambda: session.distributions(h, bad, native.PASS_DECODE)):
            with pytest.raises(native.HipError, match="not finite"):
                call()
        assert session.encode(h, good) == good_stream
        assert np.array_equal(session.decode(good_stream), good)
