"""Packed q8 / q4 block-32 projections (weight_format.rs) on the device vs
the CPU oracle running the dequantized weights.

The reference's CPU path refuses these formats (weight_format.rs:425-431);
parity is to the format's definition: every projection weight is q * scale
(pinned in test_quant_oracle.py), activations in f32. Ids bit-exact, logits
within 1e-4 of the row's largest magnitude."""
from __future__ import annotations

import numpy as np
import pytest

from esp_amd import DecoderModel, InvalidWeights, Unsupported
from esp_amd.model import LoraAdapter
from oracle import oracle, quant, st
from tests import synth

pytestmark = pytest.mark.gpu

FMT = {8: "q8-block32", 4: "q4-k32-f32-scale-f16-shared-v1"}


def _case(bits, tied, seed=5):
    cfg = synth.llama_config(2, 128, 4, 2, 256, 300, head_dim=32,
                             extra={"tie_word_embeddings": tied})
    tensors = synth.make_tensors(cfg, seed, "f32", std=0.1)
    art = quant.convert_artifact(tensors, bits)
    shapes = {n: a.shape for n, (a, _) in tensors.items()}
    ref = oracle.OracleModel(cfg, quant.dequantized_model(art, shapes, bits))
    return cfg, art, ref


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("tied", [False, True])
def test_packed_model_matches_oracle(bits, tied):
    print(f"bits {bits} tied {tied}", flush=True)
    cfg, art, ref = _case(bits, tied)
    model = DecoderModel.from_bytes(cfg, st.dump(art), FMT[bits])
    prompt = synth.uniform_ids(77, 12, cfg.vocab_size)
    kv, rkv = model.new_cache(1, 64), ref.new_cache()
    logits = model.try_forward_cached_last(prompt, kv)  # prefill: dequantized f32 GEMMs
    want = ref.forward_last(rkv, prompt)
    ids = []
    for step in range(8):  # decode: packed GEMVs
        scale = float(np.abs(want).max())
        err = float(np.abs(logits - want).max())
        assert err <= 1e-4 * scale, f"step {step}: {err} vs {scale}"
        t = oracle.argmax(want)
        assert int(np.argmax(logits)) == t
        ids.append(t)
        logits = model.try_forward_cached_last([t], kv)
        want = ref.forward_last(rkv, [t])
    dev = model.generate_greedy_device(model.new_cache(1, 64), prompt, 8, eos=[])
    assert dev == ids
    # two sequences' decode rows in one forward (multi-row path)
    kvb = model.new_cache(2, 64)
    model.forward_batch(kvb, [0, 1], [prompt, prompt[:5]])
    got = model.forward_batch(kvb, [0, 1], [[ids[0]], [ids[1]]])
    r0, r1 = ref.new_cache(), ref.new_cache()
    ref.forward_last(r0, prompt)
    ref.forward_last(r1, prompt[:5])
    for g, w in ((got[0], ref.forward_last(r0, [ids[0]])), (got[1], ref.forward_last(r1, [ids[1]]))):
        assert np.abs(g - w).max() <= 1e-4 * float(np.abs(w).max())


def test_packed_artifact_refusals():
    cfg, art, _ = _case(8, False)
    bad = dict(art)
    bad["model.norm.weight"] = (bad["model.norm.weight"][0].astype(np.float32), "F32")
    with pytest.raises(InvalidWeights, match="disagrees with declared format"):
        DecoderModel.from_bytes(cfg, st.dump(bad), FMT[8])
    bad = dict(art)
    name = "model.layers.0.mlp.down_proj.weight"
    buf = bad[name][0].copy()
    buf[-4:] = 0  # last block scale 0.0
    bad[name] = (buf, "U8")
    with pytest.raises(InvalidWeights, match="block scales are invalid"):
        DecoderModel.from_bytes(cfg, st.dump(bad), FMT[8])
    bad = dict(art)
    bad[name] = (art[name][0][:-4].copy(), "U8")
    with pytest.raises(InvalidWeights, match="byte count"):
        DecoderModel.from_bytes(cfg, st.dump(bad), FMT[8])
    bad = dict(art)
    t = synth.make_tensors(cfg, 5, "f32")
    bad[name] = t[name]
    with pytest.raises(InvalidWeights, match="unpacked projection"):
        DecoderModel.from_bytes(cfg, st.dump(bad), FMT[8])
    ad = LoraAdapter(4, 8.0, ["q_proj"], st.dump({}))
    with pytest.raises(Unsupported, match="LoRA"):
        DecoderModel.from_bytes(cfg, st.dump(art), FMT[8], adapters=[ad])


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("n", [40, 1100])
def test_packed_prefill_blocks_match_oracle(bits, n):
    """Prefill of 16+ rows (tiled MFMA attention) and of 1024+ rows (the
    LDS-streamed GEMM form): packed projections in doubled-K bf16 form on
    the matrix cores, logits within 1e-4 of the row's largest magnitude."""
    print(f"bits {bits} rows {n}", flush=True)
    cfg, art, ref = _case(bits, False, seed=9)
    model = DecoderModel.from_bytes(cfg, st.dump(art), FMT[bits])
    prompt = synth.uniform_ids(13, n, cfg.vocab_size)
    got = model.try_forward_cached_last(prompt, model.new_cache(1, n + 8))
    want = ref.forward_last(ref.new_cache(), prompt)
    assert np.abs(got - want).max() <= 1e-4 * float(np.abs(want).max())
    assert int(np.argmax(got)) == oracle.argmax(want)


@pytest.mark.parametrize("bits", [8, 4])
def test_packed_prefill_split_k_matches_oracle(bits):
    """1100 rows at hidden 1024 / FFN 2048: the doubled-K projections split
    K (four splits for down_proj, two for gate/up), so whole splits fall in
    the second half of the doubled K, where the lo products are skipped."""
    print(f"bits {bits} split-K packed prefill", flush=True)
    cfg = synth.llama_config(2, 1024, 8, 2, 2048, 300, head_dim=128)
    tensors = synth.make_tensors(cfg, 9, "f32", std=0.05)
    art = quant.convert_artifact(tensors, bits)
    shapes = {n: a.shape for n, (a, _) in tensors.items()}
    ref = oracle.OracleModel(cfg, quant.dequantized_model(art, shapes, bits))
    model = DecoderModel.from_bytes(cfg, st.dump(art), FMT[bits])
    prompt = synth.uniform_ids(13, 1100, cfg.vocab_size)
    got = model.try_forward_cached_last(prompt, model.new_cache(1, 1108))
    want = ref.forward_last(ref.new_cache(), prompt)
    assert np.abs(got - want).max() <= 1e-4 * float(np.abs(want).max())
    assert int(np.argmax(got)) == oracle.argmax(want)


@pytest.mark.parametrize("bits", [8, 4])
def test_packed_decode_wide_ffn_matches_oracle(bits):
    """FFN 14336 (the C3 width): the packed down_proj GEMV splits K over
    eight waves. Greedy decode logits within 1e-4 of the row's largest
    magnitude, ids exact, device loop ids equal to the host loop's."""
    print(f"bits {bits} FFN 14336 packed decode", flush=True)
    cfg = synth.llama_config(2, 128, 4, 2, 14336, 300, head_dim=32)
    tensors = synth.make_tensors(cfg, 21, "f32", std=0.05)
    art = quant.convert_artifact(tensors, bits)
    shapes = {n: a.shape for n, (a, _) in tensors.items()}
    ref = oracle.OracleModel(cfg, quant.dequantized_model(art, shapes, bits))
    model = DecoderModel.from_bytes(cfg, st.dump(art), FMT[bits])
    prompt = synth.uniform_ids(31, 10, cfg.vocab_size)
    kv, rkv = model.new_cache(1, 32), ref.new_cache()
    logits = model.try_forward_cached_last(prompt, kv)
    want = ref.forward_last(rkv, prompt)
    ids = []
    for step in range(6):
        err = float(np.abs(logits - want).max())
        assert err <= 1e-4 * float(np.abs(want).max()), f"step {step}: {err}"
        t = oracle.argmax(want)
        assert int(np.argmax(logits)) == t
        ids.append(t)
        logits = model.try_forward_cached_last([t], kv)
        want = ref.forward_last(rkv, [t])
    assert model.generate_greedy_device(model.new_cache(1, 32), prompt, 6, eos=[]) == ids
