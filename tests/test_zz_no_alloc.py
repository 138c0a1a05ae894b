"""ge_forward_noalloc (no device allocation; the library's scratch array) against ge_forward, the
entry point it varies: bitwise equal pooled vectors on two calls in a row, the second with a
smaller pack, for models without and with the per-layer-input branch and split-precision layers;
packs beyond the array's capacity are refused with a clear error."""
import numpy as np
import pytest

import gemma_embed as ge

pytestmark = pytest.mark.gpu


def packs(vocab):
    big = [ge.synth_tokens(s, 2, vocab, n).tolist() for s, n in ((91, 300), (92, 17), (93, 64), (94, 1))]
    small = [ge.synth_tokens(s, 2, vocab, n).tolist() for s, n in ((95, 9), (96, 40))]
    return big, small


@pytest.mark.parametrize("which", ["config2", "real_shapes"])
def test_no_alloc_forward_matches_forward(which, config2_gguf, real_shapes_gguf):
    path = config2_gguf if which == "config2" else real_shapes_gguf
    m = ge.EmbeddingModel.load(path)
    try:
        ctx = m.context
        for seqs in packs(262144):
            print(f"{which}: pack of {sum(map(len, seqs))} tokens in {len(seqs)} texts", flush=True)
            want, _ = ctx.forward(seqs)
            got, secs = ctx.forward_noalloc(seqs)
            assert secs > 0
            assert np.array_equal(got, want)
            again, _ = ctx.forward_noalloc(seqs)  # the array keeps the last call's contents
            assert np.array_equal(again, want)
        # the context's own staged batch is untouched by a no-allocation call
        big, small = packs(262144)
        ctx.batch_stage(big)
        ctx.forward_noalloc(small)
        ctx.batch_run()
        want, _ = ctx.forward(big)
        assert np.array_equal(ctx.batch_read(), want)
    finally:
        m.close()


def test_no_alloc_forward_refuses_what_does_not_fit(config2_gguf):
    m = ge.EmbeddingModel.load(config2_gguf)
    try:
        ctx = m.context
        too_big = [ge.synth_tokens(97, 2, 262144, 3000).tolist()]  # ~72 MB of workspace at d 768
        with pytest.raises(ge.GemmaEmbedError) as e:
            ctx.forward_noalloc(too_big)
        assert e.value.code == ge.GE_ERR_INVALID and "scratch" in e.value.message
        split_size = [too_big[0] + too_big[0][:1096]]  # 4096 tokens: refused whatever its workspace
        with pytest.raises(ge.GemmaEmbedError) as e:
            ctx.forward_noalloc(split_size)
        assert e.value.code == ge.GE_ERR_INVALID and "below 4096" in e.value.message
        for n in (2600, 500):  # near the array's limit at config 2's widths, then a small pack
            ok, _ = ctx.forward_noalloc([too_big[0][:n]])
            want, _ = ctx.forward([too_big[0][:n]])
            assert np.array_equal(ok, want), n
    finally:
        m.close()
