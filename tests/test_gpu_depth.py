"""HIP path vs the CPU oracle at the full depth of BASELINE configs[1] and
every layer of the 1B shape (16) and of the 8B shape with its
LoRA (32), prompt prefill then decode steps, logits within the north star's
bf16 tolerance |a - b| <= 1e-2 + 2e-2 |b| of the oracle's f32 corridor.

Depth matters for the cache's precision: error from rounding keys and
values grows with the layers it passes through. The default f32 cache is
checked at both depths; the half-precision cache (esp_kv_create_ex,
ESP_KV_F16) at the 1B depth, where a CPU emulation kept it within 0.32-0.44
of the bound (at the 8B depth the same emulation put it at 1.3-1.6x)."""
import numpy as np
import pytest

from esp_amd import DecoderModel
from esp_amd.model import LoraAdapter
from oracle import oracle, st
from tests import synth
from tests.test_gpu_wide import _close_bf16, _err, _lora

pytestmark = pytest.mark.gpu


def _run(model, ref, cfg, kv_dtype, prompt, steps, ctx):
    kv, rkv = model.new_cache(1, ctx, kv_dtype), ref.new_cache(ctx)
    got = model.try_forward_cached_last(prompt, kv)
    want = ref.forward_last(rkv, prompt)
    assert _close_bf16(got, want), ("prefill", kv_dtype, _err(got, want))
    for step in range(steps):
        t = oracle.argmax(want)
        got = model.try_forward_cached_last([t], kv)
        want = ref.forward_last(rkv, [t])
        assert _close_bf16(got, want), (step, kv_dtype, _err(got, want))


@pytest.mark.timeout(900)
def test_c2_full_depth_matches_oracle():
    """16 layers, hidden 2048, 32 q / 8 kv heads (hd 64), ffn 8192, vocab
    128256, tied head: a 384-token prompt and 4 greedy steps, with the f32
    and the half-precision cache."""
    cfg = synth.llama_config(16, 2048, 32, 8, 8192, 128256, head_dim=64, theta=500000.0,
                             max_pos=512, extra={"tie_word_embeddings": True})
    tensors = synth.make_tensors(cfg, 211, "bf16", fast=True)
    print("c2 depth: loading", flush=True)
    model = DecoderModel.from_bytes(cfg, st.dump_buffer(tensors), "bf16")
    ref = oracle.OracleModel(cfg, tensors)
    prompt = synth.uniform_ids(212, 384, cfg.vocab_size)
    for kv_dtype in ("f32", "f16"):
        print(f"c2 depth: {kv_dtype} cache", flush=True)
        _run(model, ref, cfg, kv_dtype, prompt, 4, 400)


@pytest.mark.timeout(1200)
def test_c3_full_depth_lora_matches_oracle():
    """32 layers, hidden 4096, 32 q / 8 kv heads (hd 128), ffn 14336, vocab
    128256, unmerged LoRA r16 alpha 32 on q/v: a 256-token prompt and 3
    greedy steps on the default f32 cache, against the oracle's merged-LoRA
    forward."""
    cfg = synth.llama_config(32, 4096, 32, 8, 14336, 128256, head_dim=128, theta=500000.0,
                             max_pos=512)
    tensors = synth.make_tensors(cfg, 313, "bf16", fast=True)
    ad = _lora(cfg, 7)
    print("c3 depth: loading", flush=True)
    model = DecoderModel.from_bytes(cfg, st.dump_buffer(tensors), "bf16",
                                    adapters=[LoraAdapter(16, 32.0, ["q_proj", "v_proj"],
                                                          st.dump(ad))])
    merged = oracle.apply_lora(cfg, tensors, {"rank": 16, "alpha": 32.0,
                                              "targets": ["q_proj", "v_proj"], "tensors": ad})
    del tensors
    ref = oracle.OracleModel(cfg, merged)
    prompt = synth.uniform_ids(314, 256, cfg.vocab_size)
    print("c3 depth: f32 cache", flush=True)
    _run(model, ref, cfg, "f32", prompt, 3, 300)
