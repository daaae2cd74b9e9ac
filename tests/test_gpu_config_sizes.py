"""Parity at the benchmark configurations' full sizes, through the C ABI.

* Full probability-model forward, 12 codebooks x 2580 frames (30 s), batch 3:
  the decode-side pass (one persistent frame-step launch per step, every lane
  up to context position 859, i.e. 14 key blocks of 64) returns the encode-side
  pass's distributions bit for bit at all 30,960 positions, on the reference
  geometry and on the 1024-wide one; the reference geometry's distributions
  equal the oracle's everywhere and its GPU stream equals the oracle's
  pack_normal bytes.
* Context rollover on the reference geometry at the reference test's shapes
  (tests/metal_optimized.cpp:255-261,519-524): frame steps, then the 256-frame
  replay, then frame steps resuming at context position 256.
* Long lanes on shallow stacks of the frame kernel's widths, every position
  against the oracle (block boundaries 63/64/65, 128, 256).
* Causal attention alone, 16 heads x 64, batch 3, T in {256, 1290, 2580}:
  the one-query decode mode on every sequence and the causal prefill on
  queries 0, 63, 64, 65, T-1 and 20 random ones per sequence.
"""
import concurrent.futures
import os

import numpy as np
import pytest

from tsac_hip.synthetic import REFERENCE, WIDE, Geometry, bf16_bits, pattern_tokens, random_model, random_tokens

pytestmark = pytest.mark.gpu


def _threads():
    return max(1, min(3, len(os.sched_getaffinity(0))))


@pytest.fixture(scope="module")
def native():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    from tsac_hip import native

    native.library()
    return native


@pytest.fixture(scope="module")
def reference_model(native):
    model = random_model(REFERENCE, seed=1)
    hip_model = native.HipModel(model)
    yield model, hip_model
    hip_model.close()


def _oracle_both(oracle, model, h, tokens, max_symbols=None, with_stream=True):
    """Oracle distributions and pack_normal bytes, computed concurrently (each
    call is lane-parallel over at most three threads)."""
    threads = _threads()
    with concurrent.futures.ThreadPoolExecutor(2) as pool:
        d = pool.submit(lambda: oracle.model(model).distributions(h, tokens, threads=threads,
                                                                  max_symbols=max_symbols))
        s = pool.submit(lambda: oracle.model(model).pack_normal(h, tokens, threads=threads)) if with_stream \
            else None
        return d.result(), (s.result() if s else None)


def _stream_order(frames, batch, groups, books):
    """Token indices ([frame][group][book] layout) in stream order: step, book,
    lane, group (src/format/entropy.cpp:26-60), lanes of ceil(frames/batch)
    frames with the remainder spread over the first lanes (src/common/transformer.cpp:26-60)."""
    lanes = min(batch, frames)
    base, extra = divmod(frames, lanes)
    starts, lengths = [], []
    start = 0
    for lane in range(lanes):
        length = base + (1 if lane < extra else 0)
        starts.append(start)
        lengths.append(length)
        start += length
    order = []
    for step in range(max(lengths)):
        for book in range(books):
            for lane in range(lanes):
                if step < lengths[lane]:
                    for group in range(groups):
                        order.append(((starts[lane] + step) * groups + group) * books + book)
    return np.array(order, np.int64)


@pytest.mark.timeout(900)
def test_full_forward_reference_geometry_2580_frames(native, oracle, reference_model):
    """12 codebooks x 2580 frames, batch 3: encode pass == decode pass == oracle
    at every position; GPU stream == oracle pack_normal; decode recovers the tokens.
    Contexts reach 860 keys, so past 512 the temporal attention runs in halves on
    two workgroups (blocks 8-13 merged from the second half's records)."""
    from oracle import header

    model, hip_model = reference_model
    frames, batch = 2580, 3
    h = native.header(frames, batch, 1, 12)
    tokens = random_tokens(frames, 1, 12, seed=21)
    session = hip_model.session()
    try:
        encode = session.distributions(h, tokens, native.PASS_ENCODE)
        decode = session.distributions(h, tokens, native.PASS_DECODE)
        stream = session.encode(h, tokens)
        decoded = session.decode(stream)
    finally:
        session.close()
    assert np.array_equal(encode, decode), "encode-side and decode-side passes differ"
    assert np.array_equal(decoded, tokens)
    expected, expected_stream = _oracle_both(oracle, model, header(frames, batch, 1, 12), tokens)
    mismatch = np.flatnonzero(np.any(encode != expected, axis=1))
    assert mismatch.size == 0, f"{mismatch.size} positions differ from the oracle, first {mismatch[:8]}"
    assert stream == expected_stream


@pytest.mark.timeout(600)
def test_full_forward_wide_geometry_2580_frames(native, oracle):
    """The 1024-wide geometry at the same size: encode pass == decode pass at
    every position; the oracle on the first 70 steps (context positions 0..69
    of every lane)."""
    from oracle import header

    model = random_model(WIDE, seed=2)
    hip_model = native.HipModel(model)
    frames, batch = 2580, 3
    h = native.header(frames, batch, 1, 12)
    tokens = random_tokens(frames, 1, 12, seed=22)
    session = hip_model.session()
    try:
        encode = session.distributions(h, tokens, native.PASS_ENCODE)
        decode = session.distributions(h, tokens, native.PASS_DECODE)
        stream = session.encode(h, tokens)
        decoded = session.decode(stream)
    finally:
        session.close()
        hip_model.close()
    assert np.array_equal(encode, decode), "encode-side and decode-side passes differ"
    assert np.array_equal(decoded, tokens)
    prefix = 70 * 12 * batch
    expected = oracle.model(model).distributions(header(frames, batch, 1, 12), tokens, threads=_threads(),
                                                 max_symbols=prefix)
    first = _stream_order(frames, batch, 1, 12)[:prefix]
    assert np.array_equal(encode[first], expected[first])


@pytest.mark.timeout(600)
@pytest.mark.parametrize("frames,batch,groups", [(1026, 1, 1), (3074, 3, 1)])
def test_rollover_reference_geometry(native, oracle, reference_model, frames, batch, groups):
    """One codebook, lanes longer than the 1024-position context: frame steps,
    the replay of the last 256 frames, frame steps from position 256 on."""
    from oracle import header

    model, hip_model = reference_model
    h = native.header(frames, batch, groups, 1)
    tokens = pattern_tokens(frames * groups)
    session = hip_model.session()
    try:
        stream = session.encode(h, tokens)
        decoded = session.decode(stream)
        encode = session.distributions(h, tokens, native.PASS_ENCODE)
        decode = session.distributions(h, tokens, native.PASS_DECODE)
    finally:
        session.close()
    assert np.array_equal(decoded, tokens)
    assert np.array_equal(encode, decode), "encode-side and decode-side passes differ"
    expected, expected_stream = _oracle_both(oracle, model, header(frames, batch, groups, 1), tokens)
    assert np.array_equal(encode, expected)
    assert stream == expected_stream


SHALLOW = Geometry(temporal_layers=2, codebook_layers=1)
SHALLOW_WIDE = Geometry(width=1024, heads=16, head_width=64, ffn=4096, temporal_layers=2, codebook_layers=1)


@pytest.mark.timeout(300)
@pytest.mark.parametrize("geometry,frames,batch", [(SHALLOW, 300, 1), (SHALLOW, 390, 3), (SHALLOW_WIDE, 200, 2)],
                         ids=["reference-width-1x300", "reference-width-3x130", "wide-2x100"])
def test_long_lanes_every_position(native, oracle, geometry, frames, batch):
    """The frame kernel's attention past one, two and four 64-key blocks
    (BF16-rounded value sums from position 65 on, the ordered block merge),
    every position against the oracle, stream bytes too."""
    from oracle import header

    model = random_model(geometry, seed=frames)
    hip_model = native.HipModel(model)
    h = native.header(frames, batch, 1, 12)
    tokens = random_tokens(frames, 1, 12, seed=frames + 1)
    session = hip_model.session()
    try:
        encode = session.distributions(h, tokens, native.PASS_ENCODE)
        decode = session.distributions(h, tokens, native.PASS_DECODE)
        stream = session.encode(h, tokens)
        decoded = session.decode(stream)
    finally:
        session.close()
        hip_model.close()
    expected, expected_stream = _oracle_both(oracle, model, header(frames, batch, 1, 12), tokens)
    assert np.array_equal(decode, expected), "decode-side pass differs from the oracle"
    assert np.array_equal(encode, expected), "encode-side pass differs from the oracle"
    assert stream == expected_stream
    assert np.array_equal(decoded, tokens)


# ---------------------------------------------------------------- attention alone

@pytest.mark.timeout(300)
@pytest.mark.parametrize("T", [256, 1290, 2580])
def test_attention_config_sizes(native, oracle, T):
    """16 heads x 64, batch 3, Q/K/V ~ N(0, 1) rounded to BF16, scale 1/8."""
    import torch

    heads, hw, batch = 16, 64, 3
    width = heads * hw
    scale = np.float32(0.125)
    rng = np.random.default_rng(T)
    qkv = bf16_bits(rng.standard_normal((batch, T, 3 * width)).astype(np.float32))
    d_qkv = torch.from_numpy(qkv.view(np.int16).reshape(batch * T, 3 * width).copy()).cuda()
    keys = np.ascontiguousarray(qkv[:, :, width:2 * width])
    values = np.ascontiguousarray(qkv[:, :, 2 * width:])

    # Decode mode: the last position's query over the T cached keys of each sequence.
    query = np.ascontiguousarray(qkv[:, T - 1, :width])
    out = torch.empty((batch, width), dtype=torch.int16, device="cuda")
    native.attention(torch.from_numpy(query.view(np.int16).copy()).cuda(),
                     torch.from_numpy(keys.view(np.int16).copy()).cuda(),
                     torch.from_numpy(values.view(np.int16).copy()).cuda(), T * width, batch, T, heads, hw,
                     scale, False, out)
    got = out.cpu().numpy().view(np.uint16)
    for s in range(batch):
        assert np.array_equal(got[s], oracle.attention(query[s], keys[s], values[s], heads, hw, scale, False)), s

    # Prefill: every query t over keys 0..t (causal), no replay prefix.
    start = torch.arange(batch, dtype=torch.int32, device="cuda") * T
    length = torch.full((batch,), T, dtype=torch.int32, device="cuda")
    replay = torch.zeros(batch, dtype=torch.int32, device="cuda")
    causal = torch.empty((batch * T, width), dtype=torch.int16, device="cuda")
    native.attention_causal(d_qkv, heads, hw, start, length, replay, batch, T, None, scale, causal)
    got = causal.cpu().numpy().view(np.uint16).reshape(batch, T, width)
    picks = sorted(set([0, 63, 64, 65, T - 1]) | set(rng.choice(T, 20, replace=False).tolist()))
    for s in range(batch):
        for t in picks:
            expected = oracle.attention(qkv[s, t, :width], keys[s, :t + 1], values[s, :t + 1], heads, hw, scale,
                                        False)
            assert np.array_equal(got[s, t], expected), (s, t)
