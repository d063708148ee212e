"""The bench's own shapes against the CPU oracle.

bench.py times C2 (512-token prompt, 256 greedy steps at the 1B shape),
C4 (Mixtral-style, 4 layers, a 2048-row prefill, decode at ~2.1k keys) and
the C5 step (64 sequences at 1024-1200 keys: decode rows and forced
8-token blocks through the matrix-core row attention). These tests run
those shapes through the same kernels and check them against the oracle's
f32 corridor with the north star's bf16 tolerance |a - b| <= 1e-2 + 2e-2|b|;
greedy ids are checked against the oracle's argmax wherever the oracle's
own top-1 margin is wider than the tolerance allows the GPU to move it."""
import numpy as np
import pytest

from esp_amd import DecoderModel
from esp_amd.config import DecoderConfig
from oracle import oracle, st
from tests import synth

pytestmark = pytest.mark.gpu


def _err(got, want):
    return float(np.max(np.abs(got - want) / (1e-2 + 2e-2 * np.abs(want))))


def _close_bf16(got, want, what=""):
    e = _err(got, want)
    print(f"  {what} worst error / bound {e:.3f}", flush=True)
    return e <= 1.0


def _margin_ok(want, got_id):
    """The GPU's greedy id is the oracle's argmax, or the oracle ranks the
    two within what the tolerance lets logits move (2 x the bound at the
    larger of the two)."""
    top = oracle.argmax(want)
    if got_id == top:
        return True
    a, b = float(want[top]), float(want[got_id])
    return a - b <= 2 * (1e-2 + 2e-2 * max(abs(a), abs(b)))


@pytest.mark.timeout(1200)
def test_c2_bench_shape_greedy_run():
    """BASELINE configs[1] as the bench runs it: the 1B shape at full depth
    (16 layers, hidden 2048, 32 q / 8 kv, head_dim 64, ffn 8192, vocab
    128256, theta 5e5, tied head), a 512-token prompt and 256 greedy steps
    through the device loop (captured graph, chunked replay). The oracle,
    fed the GPU's ids, agrees with every id up to its top-1 margin, and the
    GPU's logits after the whole run (the 767-token prefix as one block)
    match the oracle's."""
    cfg = synth.llama_config(16, 2048, 32, 8, 8192, 128256, head_dim=64, theta=500000.0,
                             max_pos=1024, extra={"tie_word_embeddings": True})
    tensors = synth.make_tensors(cfg, 2202, "bf16", fast=True)
    print("c2 shape: loading", flush=True)
    model = DecoderModel.from_bytes(cfg, st.dump_buffer(tensors), "bf16")
    ref = oracle.OracleModel(cfg, tensors)
    prompt = synth.uniform_ids(2203, 512, cfg.vocab_size)
    print("c2 shape: device greedy loop, 256 steps", flush=True)
    ids = model.generate_greedy_device(model.new_cache(1, 800), prompt, 256, eos=[])
    assert len(ids) == 256
    rkv = ref.new_cache(800)
    want = ref.forward_last(rkv, prompt)
    moved = 0
    for i, t in enumerate(ids):
        assert _margin_ok(want, t), (i, t, oracle.argmax(want))
        moved += t != oracle.argmax(want)
        if i + 1 < len(ids):
            want = ref.forward_last(rkv, [t])
        if i % 64 == 63:
            print(f"  oracle step {i + 1}", flush=True)
    print(f"  ids off the oracle's argmax within its margin: {moved}", flush=True)
    # `want` now holds the oracle's logits after feeding ids[:-1]
    got = model.try_forward_cached_last(prompt + ids[:-1], model.new_cache(1, 800))
    assert _close_bf16(got, want, "after 767 tokens"), _err(got, want)


@pytest.mark.timeout(1200)
def test_c4_bench_shape_prefill_and_decode():
    """BASELINE configs[3] at the bench's shape: Mixtral-style, 4 layers,
    hidden 4096, 32 q / 8 kv, 8 experts of SwiGLU 14336, top-2 renormalised,
    vocab 32000; a 2048-row prefill (near-uniform routing through the
    grouped expert GEMMs) and four decode steps at 2048-2051 keys through
    the device router and expert-indexed GEMVs, each vs the oracle."""
    cfg = DecoderConfig.mixtral_style(vocab_size=32000, hidden_size=4096, intermediate_size=14336,
                                      num_hidden_layers=4, num_attention_heads=32,
                                      num_key_value_heads=8, max_position_embeddings=2176,
                                      rope_theta=1000000.0, num_experts=8, num_experts_per_tok=2,
                                      moe_intermediate_size=14336)
    tensors = synth.make_tensors(cfg, 4404, "bf16", fast=True)
    print("c4 shape: loading", flush=True)
    model = DecoderModel.from_bytes(cfg, st.dump_buffer(tensors), "bf16")
    ref = oracle.OracleModel(cfg, tensors)
    prompt = synth.uniform_ids(4405, 2048, cfg.vocab_size)
    kv, rkv = model.new_cache(1, 2112), ref.new_cache(2112)
    print("c4 shape: prefill 2048", flush=True)
    got = model.try_forward_cached_last(prompt, kv)
    want = ref.forward_last(rkv, prompt)
    assert _close_bf16(got, want, "prefill"), _err(got, want)
    for step in range(4):
        t = oracle.argmax(want)
        got = model.try_forward_cached_last([t], kv)
        want = ref.forward_last(rkv, [t])
        assert _close_bf16(got, want, f"decode {step} at {kv.position()} keys"), _err(got, want)


@pytest.mark.timeout(1200)
@pytest.mark.parametrize("kv_dtype", ["f32", "f16"])
def test_c5_bench_shape_rows_over_long_contexts(kv_dtype):
    """The C5 step's attention shapes: 64 sequences at 1024-1200 cached keys
    with the 1B shape's heads (32 q / 8 kv, head_dim 64) over a narrow
    hidden (256, two layers, so the oracle runs every sequence): one step of
    56 decode rows + 8 forced 8-token blocks, then 64 decode rows, through
    the matrix-core row attention (512 units). The last sequence's last row
    sits at the cache's final position (its keys end at max_ctx). Every
    row's logits vs the oracle run on its sequence alone."""
    n = 64
    cfg = synth.llama_config(2, 256, 32, 8, 512, 1000, head_dim=64, theta=500000.0,
                             max_pos=2048)
    tensors = synth.make_tensors(cfg, 5505, "bf16")
    model = DecoderModel.from_bytes(cfg, st.dump(tensors), "bf16")
    ref = oracle.OracleModel(cfg, tensors)
    # the last sequence ends its two steps exactly at max_ctx
    max_ctx = 1210
    lens = [1024 + (i * 37) % 177 for i in range(n - 1)] + [max_ctx - 9]
    prompts = [synth.uniform_ids(5600 + i, lens[i], cfg.vocab_size) for i in range(n)]
    kv = model.new_cache(n, max_ctx, kv_dtype)
    print(f"c5 shape: 64 prompts of 1024-1200 tokens ({kv_dtype} cache)", flush=True)
    got = model.forward_batch(kv, list(range(n)), prompts)
    rkvs = [ref.new_cache(max_ctx) for _ in range(n)]
    worst = 0.0
    for i in range(n):
        want = ref.forward_last(rkvs[i], prompts[i])
        worst = max(worst, _err(got[i], want))
    print(f"  prompts worst error / bound {worst:.3f}", flush=True)
    assert worst <= 1.0
    rng = np.random.default_rng(5507)
    blocks = [[int(x) for x in rng.integers(0, cfg.vocab_size, 8)] if i % 8 == 3
              else [int(rng.integers(0, cfg.vocab_size))] for i in range(n)]
    blocks[n - 1] = [int(x) for x in rng.integers(0, cfg.vocab_size, 8)]
    for step in range(2):
        got = model.forward_batch(kv, list(range(n)), blocks)
        worst = 0.0
        for i in range(n):
            want = ref.forward_last(rkvs[i], blocks[i])
            worst = max(worst, _err(got[i], want))
        print(f"  step {step} worst error / bound {worst:.3f}", flush=True)
        assert worst <= 1.0, step
        blocks = [[int(rng.integers(0, cfg.vocab_size))] for _ in range(n)]
    assert kv.position(n - 1) == max_ctx
