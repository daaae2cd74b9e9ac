"""The known-token pass under Limits::cache_bytes.

The batched encode pass computes whole sequences and many frames of codebook
rows ahead; with the persistent key/value caches its scratch must fit
Limits::cache_bytes, as the lookahead of the reference's Metal encoder must
(src/metal/transformer/encoding.mm:139-150, tested there at 2,300,000 bytes,
tests/metal_optimized.cpp:277-292). It shrinks its batches to fit, and where
not even one sequence and one frame step fit, the encode runs step by step on
the frame-step path, taking each token's Q15 splits from the draw. The stream
must not change: every budget here gives the unbounded encode's bytes.
"""
import numpy as np
import pytest

from tsac_hip.synthetic import Geometry, pattern_tokens, random_model

pytestmark = pytest.mark.gpu

SMALL = Geometry(width=256, heads=2, head_width=128, ffn=512, temporal_layers=2, codebook_layers=1, latent=256)


@pytest.fixture(scope="module")
def native():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    from tsac_hip import native

    native.library()
    return native


def persistent_bytes(g, frames, batch, groups, books):
    """Key/value cache bytes of the lanes (src/common/cpu_transformer.tpp:285-305)."""
    lanes = min(batch, frames)
    base, extra = divmod(frames, batch)
    contexts = groups * ((batch - extra) * min(base, g.context) + extra * min(base + 1, g.context))
    return contexts * g.temporal_layers * g.width * 4 + lanes * groups * books * g.codebook_layers * g.width * 4


@pytest.mark.parametrize("frames,batch,groups,books", [(35, 3, 2, 12), (90, 3, 1, 1), (101, 3, 1, 12),
                                                       (1030, 1, 1, 1)])
def test_encode_within_cache_limit_keeps_the_stream(native, frames, batch, groups, books):
    model = random_model(SMALL, seed=4)
    h = native.header(frames, batch, groups, books)
    tokens = pattern_tokens(frames * groups * books)
    with native.HipModel(model) as unbounded, unbounded.session() as session:
        want = session.encode(h, tokens)
        assert not session.timing()["stepwise"]  # the batched pass
    kv = persistent_bytes(SMALL, frames, batch, groups, books)
    fixed = frames * groups * (2 * SMALL.width + 2 * books)
    seen_stepwise = False
    for extra in (0, 40_000, 400_000, 2_000_000, 12_000_000):
        limits = native.Limits()
        limits.cache_bytes = kv + fixed + extra
        print(f"shape {frames}x{batch}x{groups}x{books} cache_bytes {limits.cache_bytes}", flush=True)
        with native.HipModel(model, limits=limits) as bounded, bounded.session() as session:
            got = session.encode(h, tokens)
            seen_stepwise |= session.timing()["stepwise"]
            assert got == want, extra
            assert np.array_equal(session.decode(got), tokens)
    assert seen_stepwise, "the tightest budget runs the encode step by step"


def test_cache_limit_below_the_persistent_caches_is_an_error(native):
    model = random_model(SMALL, seed=4)
    limits = native.Limits()
    limits.cache_bytes = persistent_bytes(SMALL, 90, 3, 1, 1) - 1
    h = native.header(90, 3, 1, 1)
    with native.HipModel(model, limits=limits) as bounded, bounded.session() as session:
        with pytest.raises(native.HipError, match="cache_bytes"):
            session.encode(h, pattern_tokens(90))
