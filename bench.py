"""Benchmark: llama-family decode & prefill tokens/s on one MI355X.

Headline workload ("C3"): Llama-3-8B-shape
decoder, bf16 weights (random init N(0, 0.02), synthetic) with rank-16 LoRA
(alpha 32) on q_proj and v_proj, batch 1: a 4064-token uniform-random prompt
then 64 greedy decode steps, i.e. decode at 4064-4128 (mean 4096) context.
One "step" is that whole request; `value` is decode tokens/s (the prompt's
prefill, timed separately, is subtracted). A separate 2048-token prefill is
reported as prefill tokens/s and a fraction of bf16 MFMA peak.

`decode_hbm_frac` counts BASELINE.md's algorithmic bytes per token (every
weight once in bf16 + the K/V cache once at 2 bytes per element); the
`roofline` object describes the dominant decode kernel (the SwiGLU gate/up
GEMV) from HIP events recorded on the KV handle's stream around every launch
of that kernel in an eager pass; `traffic` is its measured HBM bytes per
launch from the committed FETCH_SIZE / WRITE_SIZE counter summary.
`cpu_baseline` times the CPU restatement of esp's burn-ndarray path
(oracle/) on the same C3 decode at 4096 context on all host cores. The
other BASELINE configs (C2, C4, C5) and the widened rows are extra objects.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, AMD spec
BF16_PEAK_TFLOPS = 2516.6      # MI355X dense bf16 MFMA, AMD spec
GOLDEN = 0x9E3779B97F4A7C15


def uniform_ids(seed: int, n: int, vocab: int):
    """n token ids uniform in [0, vocab): splitmix64 outputs seed + k*gamma
    (k = 1..n) reduced mod vocab."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + np.uint64(GOLDEN) * np.arange(1, n + 1, dtype=np.uint64)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return [int(v % vocab) for v in z]


def llama_config(layers, hidden, heads, kv_heads, ffn, vocab, theta=10000.0, max_pos=2048,
                 extra=None):
    from esp_amd.config import DecoderConfig
    raw = {"architectures": ["LlamaForCausalLM"], "model_type": "llama",
           "hidden_size": hidden, "intermediate_size": ffn, "num_hidden_layers": layers,
           "num_attention_heads": heads, "num_key_value_heads": kv_heads,
           "max_position_embeddings": max_pos, "rms_norm_eps": 1e-5, "rope_theta": theta,
           "vocab_size": vocab, "tie_word_embeddings": False, "hidden_act": "silu"}
    raw.update(extra or {})
    return DecoderConfig.from_json_bytes(json.dumps(raw).encode())


def llama_sized_table(seed: int = 11, n: int = 128256):
    """Every single byte, then random multi-byte tokens: ASCII words and
    punctuation, quotes and backslashes, whole and split UTF-8 sequences,
    control bytes; empty entries stand for added tokens."""
    rng = np.random.default_rng(seed)
    pieces = [bytes([b]) for b in range(256)]
    ascii_ = np.frombuffer(b"abcdefghijklmnopqrstuvwxyz _-:,{}[]\"\\0123456789./", np.uint8)
    utf = ["é", "→", "日", "\U0001F600", "ü", "ß"]
    while len(pieces) < n - 256:
        k = int(min(1 + rng.geometric(0.22), 24))
        out = bytearray()
        while len(out) < k:
            r = rng.random()
            if r < 0.8:
                out.append(int(rng.choice(ascii_)))
            elif r < 0.92:
                out += utf[int(rng.integers(len(utf)))].encode()
            elif r < 0.97:
                s = utf[int(rng.integers(len(utf)))].encode()
                cut = int(rng.integers(1, len(s))) if len(s) > 1 else 1
                out += s[:cut] if rng.random() < 0.5 else s[cut:]
            else:
                out.append(int(rng.integers(0, 256)))
        pieces.append(bytes(out))
    pieces += [b""] * (n - len(pieces))
    return pieces


def c2_config(max_pos=2048):
    return llama_config(16, 2048, 32, 8, 8192, 128256, theta=500000.0, max_pos=max_pos,
                        extra={"tie_word_embeddings": True})


def c3_config(max_pos=8192):
    return llama_config(32, 4096, 32, 8, 14336, 128256, theta=500000.0, max_pos=max_pos)


C3_LORA = dict(lora_rank=16, lora_targets=["q_proj", "v_proj"], lora_a_std=0.02,
               lora_b_std=0.01, lora_scale=2.0)


def device_sync() -> None:
    """hipDeviceSynchronize through the HIP runtime the library links."""
    import ctypes as C
    global _HIP
    if "_HIP" not in globals():
        _HIP = C.CDLL("libamdhip64.so.7")
    assert _HIP.hipDeviceSynchronize() == 0


def greedy_self_check(model, kv, prompt, dev_ids, n: int = 8) -> None:
    """Consistency of a timed device greedy loop (one captured decode step
    replayed per token, the argmax in the head kernel): its first `n` ids
    equal a host loop of eager forwards over the same prompt with a host
    argmax (lowest id on ties, as the head kernel's). Runs after the timed
    region; raises on a mismatch."""
    import numpy as np
    kv.reset(0)
    logits = model.try_forward_cached_last(prompt, kv)
    host = []
    for _ in range(n):
        t = int(np.argmax(logits))
        host.append(t)
        logits = model.try_forward_cached_last([t], kv)
    if host != [int(x) for x in dev_ids[:n]]:
        raise RuntimeError(f"device greedy ids {list(dev_ids[:n])} differ from the host loop's {host}")


def decode_bytes(cfg, ctx: int, kv_bytes_per_elem: int = 2, lora_rank: int = 0,
                 lora_targets=()) -> dict:
    """Algorithmic HBM bytes of one batch-1 decode step at context `ctx`:
    every weight once (bf16) + the K/V cache once (kv_bytes_per_elem bytes
    per element; BASELINE.md counts 2) + LoRA A/B (bf16)."""
    H, L, F, V = cfg.hidden_size, cfg.num_hidden_layers, cfg.intermediate_size, cfg.vocab_size
    qw, kvw = cfg.query_width(), cfg.kv_heads() * cfg.head_dim()
    lora = 0
    for t in lora_targets:
        outf = qw if t == "q_proj" else kvw
        lora += lora_rank * (H + outf) * 2
    layer_w = (H * (qw + 2 * kvw) + H * qw + 3 * H * F) * 2 + lora
    head_w = V * H * 2
    kv = 2 * L * kvw * ctx * kv_bytes_per_elem
    return {"gemv_weights": L * layer_w + head_w, "kv": kv, "total": L * layer_w + head_w + kv}


def mlp_gemv_bytes(cfg) -> int:
    """Algorithmic bytes of one decode SwiGLU GEMV launch: gate and up rows
    (bf16, F x H each), the input row and RMSNorm weight (f32, H each), the
    activation row written (f32, F)."""
    H, F = cfg.hidden_size, cfg.intermediate_size
    return 2 * F * H * 2 + 2 * H * 4 + F * 4


def profile_value(key: str, name: str = "decode_gemv_mlp_c3_traffic.md"):
    """A `key: value` line of a committed counter summary (profiles/), or None."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        for line in open(path):
            if line.startswith(key + ":"):
                return float(line.split(":")[1])
    except OSError:
        pass
    return None


def measured_traffic(name: str = "decode_gemv_mlp_c3_traffic.md"):
    """HBM bytes per launch of the roofline kernel from the committed
    FETCH_SIZE / WRITE_SIZE counter summary (profiles/), or None."""
    v = profile_value("traffic_bytes_per_launch", name)
    return int(v) if v is not None else None


def traffic_run(steps: int = 8) -> None:
    """Workload for the counter passes (FETCH_SIZE, WRITE_SIZE, MFMA busy):
    one plain device-to-device copy of known size (the calibration
    dispatch), then on the C3 model a 2048-token prefill (the headline
    prefill's GEMMs and attention), a 2016-token continuation over that
    cache, and `steps` eager decode steps at 4064-4072 context (every decode
    kernel of the headline, the SwiGLU GEMV among them)."""
    import torch
    from esp_amd import DecoderModel
    n = 64 << 20
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    cfg = c3_config()
    model = DecoderModel.synthetic(cfg, seed=4321, std=0.02, fmt="bf16", **C3_LORA)
    kv = model.new_cache(1, 4064 + steps)
    prompt = uniform_ids(7, 4064, cfg.vocab_size)
    print("traffic: model ready", file=sys.stderr, flush=True)
    model.try_forward_cached_last(prompt[:2048], kv)
    model.try_forward_cached_last(prompt[2048:], kv)
    print("traffic: prefill done", file=sys.stderr, flush=True)
    for i in range(steps):
        model.try_forward_cached_last([i + 1], kv)
    model.close()
    print(json.dumps({"copy_bytes": n * 4, "mlp_gemv_bytes": mlp_gemv_bytes(cfg),
                      "prefill_rows": [2048, 2016], "decode_steps": steps}), flush=True)


def prefill_flops(cfg, S: int) -> float:
    H, L, F, V = cfg.hidden_size, cfg.num_hidden_layers, cfg.intermediate_size, cfg.vocab_size
    qw, kvw, hd, nq = cfg.query_width(), cfg.kv_heads() * cfg.head_dim(), cfg.head_dim(), \
        cfg.num_attention_heads
    gemm = 2.0 * S * L * (H * (qw + 2 * kvw) + H * qw + 3 * H * F)
    attn = 2.0 * 2.0 * L * nq * hd * S * (S + 1) / 2
    head = 2.0 * H * V
    return gemm + attn + head


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(cfg, ctx: int = 4096, decode_runs: int = 7, prefill_len: int = 32,
                 prefill_runs: int = 5) -> dict:
    """The oracle (CPU restatement of esp's f32 corridor: bf16 weights widened
    to f32 on the fly, head on the last position) on every host core: the
    whole C3 model (32 layers, untied head) decoding one token at `ctx`
    context over a K/V cache filled from the seed, median of `decode_runs`
    single-token steps after one warm-up; and a `prefill_len`-token prompt
    on an empty cache, median of `prefill_runs`. LoRA is left out: the
    reference merges adapters into the weights at load (lora.rs:93-97), so
    its decode cost is the base model's."""
    from oracle import oracle
    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    oracle.set_threads(threads)
    H, F, V = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size
    qw, kvw = cfg.query_width(), cfg.kv_heads() * cfg.head_dim()
    tensors = {}
    seed = 1

    def put(name, shape, one=False):
        nonlocal seed
        if one:
            tensors[name] = (np.ones(shape, np.float32), "F32")
        else:
            seed += 1
            tensors[name] = (oracle.fill_normal(seed, int(np.prod(shape)), 0.02, True)
                             .reshape(shape), "BF16")

    t0 = time.perf_counter()
    put("model.embed_tokens.weight", (V, H))
    put("model.norm.weight", (H,), True)
    put("lm_head.weight", (V, H))
    for l in range(cfg.num_hidden_layers):
        p = f"model.layers.{l}."
        put(p + "input_layernorm.weight", (H,), True)
        put(p + "post_attention_layernorm.weight", (H,), True)
        put(p + "self_attn.q_proj.weight", (qw, H))
        put(p + "self_attn.k_proj.weight", (kvw, H))
        put(p + "self_attn.v_proj.weight", (kvw, H))
        put(p + "self_attn.o_proj.weight", (H, qw))
        put(p + "mlp.gate_proj.weight", (F, H))
        put(p + "mlp.up_proj.weight", (F, H))
        put(p + "mlp.down_proj.weight", (H, F))
    m = oracle.OracleModel(cfg, tensors, rope_max_pos=ctx + decode_runs + 8)
    print(f"cpu_baseline: weights ready in {time.perf_counter() - t0:.1f} s on {threads} threads",
          file=sys.stderr, flush=True)
    kv = m.new_cache(ctx + decode_runs + 8)
    kv.fill_synthetic(ctx, 5)
    m.forward_last(kv, [1])  # warm-up (position ctx)
    dec = []
    for i in range(decode_runs):
        t1 = time.perf_counter()
        m.forward_last(kv, [(i * 7919) % V])
        dec.append(time.perf_counter() - t1)
    t_dec = sorted(dec)[len(dec) // 2]
    pre = []
    prompt = uniform_ids(77, prefill_len, V)
    for _ in range(prefill_runs):
        kvp = m.new_cache(prefill_len + 8)
        t1 = time.perf_counter()
        m.forward_last(kvp, prompt)
        pre.append(time.perf_counter() - t1)
        del kvp
    t_pre = sorted(pre)[len(pre) // 2]
    return {"value": round(1.0 / t_dec, 4), "unit": "tokens/s (decode, batch 1)",
            "cores": threads, "kind": "port",
            "sample": f"whole C3 model ({cfg.num_hidden_layers} layers, hidden {H}, ffn {F}, "
                      f"vocab {V}, bf16 weights widened to f32), one decode token at context {ctx + 1}-"
                      f"{ctx + decode_runs} over a seeded synthetic K/V cache, median of "
                      f"{decode_runs} steps; CPU restatement of esp's burn-ndarray path, "
                      f"OpenMP over {threads} threads",
            "cpu_model": cpu_model(), "nproc": os.cpu_count(),
            "decode_ms_per_token": round(t_dec * 1e3, 2),
            "prefill_tokens_per_s": round(prefill_len / t_pre, 3),
            "prefill_sample": f"{prefill_len}-token prompt on an empty cache, median of "
                              f"{prefill_runs} runs"}


def c3_headline(steps: int, warmup: int) -> dict:
    """Llama-3-8B shape bf16 with rank-16 LoRA (alpha 32)
    on q_proj and v_proj. One step = one request: a 4064-token prompt and 64
    greedy decode tokens through the device loop (one captured decode step
    replayed per token); decode time = step time minus the prompt's prefill
    (the same 4064 tokens timed alone). Plus a separate 2048-token prefill
    and the roofline pass over the dominant decode kernel."""
    from esp_amd import DecoderModel
    from esp_amd.model import profile_enable, profile_read
    cfg = c3_config()
    model = DecoderModel.synthetic(cfg, seed=4321, std=0.02, fmt="bf16", **C3_LORA)
    prompt = uniform_ids(7, 4064, cfg.vocab_size)
    n_dec = 64
    kv = model.new_cache(1, 4064 + n_dec)
    pre = uniform_ids(8, 2048, cfg.vocab_size)

    def prefill(ids):
        kv.reset(0)
        t0 = time.perf_counter()
        model.try_forward_cached_last(ids, kv)
        return time.perf_counter() - t0

    dev = {}

    def gen():
        t0 = time.perf_counter()
        out = model.generate_greedy_device(kv, prompt, n_dec, eos=[])
        assert len(out) == n_dec
        dev["ids"] = out
        return time.perf_counter() - t0

    for _ in range(max(1, warmup)):
        gen()
        prefill(pre)
    device_sync()
    t0 = time.perf_counter()
    t_gen = [gen() for _ in range(steps)]
    device_sync()
    el = time.perf_counter() - t0
    t_p4 = sorted(prefill(prompt) for _ in range(steps))[steps // 2]
    t_p2 = sorted(prefill(pre) for _ in range(steps))[steps // 2]
    greedy_self_check(model, kv, prompt, dev["ids"])
    tg = sorted(t_gen)[steps // 2]
    t_dec = (tg - t_p4) / (n_dec - 1)
    ctx = 4064 + n_dec // 2
    db = decode_bytes(cfg, ctx, 2, **{k: C3_LORA[k] for k in ("lora_rank", "lora_targets")})
    own = decode_bytes(cfg, ctx, 4, **{k: C3_LORA[k] for k in ("lora_rank", "lora_targets")})
    fl = prefill_flops(cfg, 2048) + 2.0 * 2048 * 32 * 16 * (4096 + 4096 + 4096 + 1024)  # + LoRA
    # roofline pass: HIP events around every launch of the SwiGLU GEMV
    # family over 16 eager decode steps at the same context
    kv.reset(0)
    model.try_forward_cached_last(prompt, kv)
    profile_enable("gemv_mlp", True)
    before = profile_read("gemv_mlp")
    for i in range(16):
        model.try_forward_cached_last([i + 1], kv)
    after = profile_read("gemv_mlp")
    profile_enable("gemv_mlp", False)
    launches = after[0] - before[0]
    ms = after[1] - before[1]
    gbs = mlp_gemv_bytes(cfg) * launches / (ms / 1e3) / 1e9
    model.close()
    return {
        "value": round(1.0 / t_dec, 2), "ms_per_step": round(tg * 1e3, 3),
        "timed_region_s": round(el, 3),
        "decode_ms_per_token": round(t_dec * 1e3, 4),
        "decode_hbm_frac": round(db["total"] / t_dec / 1e9 / HBM_PEAK_GBS, 4),
        "decode_bytes_per_token": db["total"],
        "decode_hbm_frac_own_bytes": round(own["total"] / t_dec / 1e9 / HBM_PEAK_GBS, 4),
        "decode_own_bytes_per_token": own["total"],
        "prefill_tokens_per_s": round(2048 / t_p2, 1),
        "prefill_2048_ms": round(t_p2 * 1e3, 3),
        "prefill_mfma_frac": round(fl / t_p2 / 1e12 / BF16_PEAK_TFLOPS, 4),
        "prompt_4064_prefill_ms": round(t_p4 * 1e3, 3),
        "roofline": {"bound": "hbm",
                     "kernel": "decode_gemv_k<bf16, SWIGLU> (C3 gate+up projections, fused "
                               "RMSNorm: 2 x 14336 x 4096 bf16 weights per launch)",
                     "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "algorithmic_bytes": mlp_gemv_bytes(cfg), "launches": launches,
                     "avg_launch_us": round(ms / max(1, launches) * 1e3, 3),
                     "timing": "HIP events around each launch on the cache's stream over 16 eager "
                               "decode steps: the span includes the dispatch gap after the previous "
                               "kernel",
                     **kernel_trace_frac(cfg)},
    }


def kernel_trace_frac(cfg) -> dict:
    """The roofline kernel's fraction on its rocprofv3 kernel-trace duration
    (the committed summary of the counter runs: kernel time only, no dispatch
    gap), beside the bench's own HIP-event figure."""
    us = profile_value("kernel_trace_avg_us")
    if not us:
        return {}
    gbs = mlp_gemv_bytes(cfg) / (us * 1e-6) / 1e9
    return {"kernel_trace_avg_us": us, "kernel_trace_frac": round(gbs / HBM_PEAK_GBS, 4)}


def c2_bench(steps: int, warmup: int, prompt_len: int = 512, n_decode: int = 256) -> dict:
    """Llama-3.2-1B shape bf16, batch 1: a 512-token
    prompt then 256 greedy decode steps (device loop); decode tokens/s with
    the prefill subtracted, and the prefill rate."""
    from esp_amd import DecoderModel
    cfg = c2_config()
    model = DecoderModel.synthetic(cfg, seed=1234, std=0.02, fmt="bf16")
    prompt = uniform_ids(42, prompt_len, cfg.vocab_size)
    kv = model.new_cache(1, prompt_len + n_decode)

    dev = {}

    def gen():
        t0 = time.perf_counter()
        out = model.generate_greedy_device(kv, prompt, n_decode, eos=[])
        assert len(out) == n_decode
        dev["ids"] = out
        return time.perf_counter() - t0

    def prefill():
        kv.reset(0)
        t0 = time.perf_counter()
        model.try_forward_cached_last(prompt, kv)
        return time.perf_counter() - t0

    for _ in range(max(1, warmup)):
        gen()
        prefill()
    tg = sorted(gen() for _ in range(steps))[steps // 2]
    tp = sorted(prefill() for _ in range(steps))[steps // 2]
    greedy_self_check(model, kv, prompt, dev["ids"])
    t_dec = (tg - tp) / (n_decode - 1)
    db = decode_bytes(cfg, prompt_len + n_decode // 2)
    model.close()
    return {"workload": "C2: Llama-3.2-1B shape bf16, 512-token prefill + 256 greedy decode "
                        "steps, batch 1 (BASELINE configs[1])",
            "decode_tokens_per_s": round(1.0 / t_dec, 2),
            "decode_ms_per_token": round(t_dec * 1e3, 4),
            "decode_hbm_frac": round(db["total"] / t_dec / 1e9 / HBM_PEAK_GBS, 4),
            "decode_bytes_per_token": db["total"],
            "prefill_tokens_per_s": round(prompt_len / tp, 1),
            "prefill_ms": round(tp * 1e3, 3),
            "prefill_mfma_frac": round(prefill_flops(cfg, prompt_len) / tp / 1e12 / BF16_PEAK_TFLOPS, 4)}


def packed_decode_bytes(cfg, ctx: int, bits: int) -> dict:
    """Algorithmic HBM bytes of one batch-1 decode step with packed
    projections (weight_format.rs:138-223): bits/8 bytes per weight plus one
    f32 scale per 32, the head packed too (untied), the K/V cache (f32)."""
    H, L, F, V = cfg.hidden_size, cfg.num_hidden_layers, cfg.intermediate_size, cfg.vocab_size
    qw, kvw = cfg.query_width(), cfg.kv_heads() * cfg.head_dim()
    per = bits / 8 + 4 / 32
    layer_w = (H * (qw + 2 * kvw) + H * qw + 3 * H * F) * per
    head_w = V * H * per
    kv = 2 * L * kvw * ctx * 4
    return {"gemv_weights": int(L * layer_w + head_w), "kv": kv,
            "total": int(L * layer_w + head_w + kv)}


def c3_packed_bench(bits: int) -> dict:
    """The C3 shape (Llama-3-8B, no LoRA) with packed q8 / q4 block-32
    projections: batch-1 greedy decode at ~4.1k context. Decode time per
    token is the difference of two device loops (16 and 80 new tokens) over
    the same 4064-token prompt, so the prompt's prefill cancels."""
    from esp_amd import DecoderModel
    cfg = c3_config()
    fmt = "q8-block32" if bits == 8 else "q4-block32"
    model = DecoderModel.synthetic(cfg, seed=4321, std=0.02, fmt=fmt)
    prompt = uniform_ids(7, 4064, cfg.vocab_size)
    kv = model.new_cache(1, 4064 + 80)

    dev = {}

    def gen(n):
        t0 = time.perf_counter()
        out = model.generate_greedy_device(kv, prompt, n, eos=[])
        assert len(out) == n
        dev["ids"] = out
        return time.perf_counter() - t0

    gen(16)
    t16, t80 = gen(16), gen(80)
    t_dec = (t80 - t16) / 64
    greedy_self_check(model, kv, prompt, dev["ids"])
    db = packed_decode_bytes(cfg, 4064 + 48, bits)
    # 2048-token prefill: doubled-K bf16 projections on the matrix cores
    kvp = model.new_cache(1, 2048 + 8)
    t_pre = []
    for _ in range(3):
        kvp.reset(0)
        t0 = time.perf_counter()
        model.try_forward_cached_last(prompt[:2048], kvp)
        t_pre.append(time.perf_counter() - t0)
    t_pre = min(t_pre[1:])
    res = {"workload": f"C3 shape (Llama-3-8B, no LoRA) with {fmt} projections; batch-1 greedy "
                       "decode at 4080-4144 context; separate 2048-token prefill",
           "decode_tokens_per_s": round(1.0 / t_dec, 2),
           "decode_ms_per_token": round(t_dec * 1e3, 4),
           "decode_hbm_frac": round(db["total"] / t_dec / 1e9 / HBM_PEAK_GBS, 4),
           "decode_bytes_per_token": db["total"],
           "prefill_2048_ms": round(t_pre * 1e3, 2),
           "prefill_2048_tokens_per_s": round(2048 / t_pre, 1),
           "weight_bytes": model.weight_bytes()}
    model.close()
    return res


def synthetic_layer_artifacts(cfg, seed: int = 9):
    """bf16 artifacts of cfg's dense block in esp's streamed layout: the
    shared artifact (embedding, final norm, head) and one safetensors
    artifact per layer. Values are uniform bf16 in [2^-7, 2^-6); every layer
    carries the same bytes under its own names."""
    from esp_amd.streaming import layer_tensor_names, pack
    rng = np.random.default_rng(seed)
    H, F, V = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size
    qw, kvw = cfg.query_width(), cfg.kv_heads() * cfg.head_dim()
    shapes = {"input_layernorm.weight": (H,), "post_attention_layernorm.weight": (H,),
              "self_attn.q_proj.weight": (qw, H), "self_attn.k_proj.weight": (kvw, H),
              "self_attn.v_proj.weight": (kvw, H), "self_attn.o_proj.weight": (H, qw),
              "mlp.gate_proj.weight": (F, H), "mlp.up_proj.weight": (F, H),
              "mlp.down_proj.weight": (H, F)}
    assert set(shapes) == set(layer_tensor_names(cfg))

    def vals(shape):
        return rng.integers(0x3c00, 0x3c80, size=int(np.prod(shape)), dtype=np.uint16).tobytes()

    data = {k: vals(v) for k, v in shapes.items()}
    layers = [pack([(f"model.layers.{l}.{k}", "BF16", v, data[k]) for k, v in shapes.items()])
              for l in range(cfg.num_hidden_layers)]
    shared = pack([("model.embed_tokens.weight", "BF16", (V, H), vals((V, H))),
                   ("model.norm.weight", "BF16", (H,), vals((H,))),
                   ("lm_head.weight", "BF16", (V, H), vals((V, H)))])
    return shared, layers


def h2d_gbs(nbytes: int = 512 << 20, reps: int = 8) -> float:
    """Pinned host-to-device copy rate of this box: hipMemcpyAsync from
    hipHostMalloc memory on one stream, through the HIP runtime the library
    itself links."""
    import ctypes as C
    hip = C.CDLL("libamdhip64.so.7")  # the runtime libesp_hip.so is linked to
    h, d = C.c_void_p(), C.c_void_p()
    assert hip.hipHostMalloc(C.byref(h), C.c_size_t(nbytes), 0) == 0
    assert hip.hipMalloc(C.byref(d), C.c_size_t(nbytes)) == 0
    try:
        def copy():
            assert hip.hipMemcpyAsync(d, h, C.c_size_t(nbytes), 1, None) == 0  # host to device

        for _ in range(2):
            copy()
        assert hip.hipDeviceSynchronize() == 0
        t0 = time.perf_counter()
        for _ in range(reps):
            copy()
        assert hip.hipDeviceSynchronize() == 0
        return nbytes * reps / (time.perf_counter() - t0) / 1e9
    finally:
        hip.hipFree(d)
        hip.hipHostFree(h)


def c3_stream_bench() -> dict:
    """The C3 shape (Llama-3-8B, bf16, no LoRA) with every layer streamed
    from host artifacts through a LayerSource (esp.layer-weights layout):
    each forward reads all 32 layers (~14 GB) and stages them into HBM on a
    copy stream while the previous layer computes. Bound: the host link.
    Then the same model with a device layer cache holding every layer."""
    from esp_amd import DecoderModel
    from esp_amd.streaming import ArtifactSource, StreamingOptions
    cfg = c3_config()
    shared, layers = synthetic_layer_artifacts(cfg)
    per_forward = sum(len(x) for x in layers)
    opts = StreamingOptions(max_layer_bytes=max(len(x) for x in layers),
                            max_shared_bytes=len(shared))
    model = DecoderModel.from_layer_source(cfg, shared, ArtifactSource(layers), opts, "bf16")
    prompt = uniform_ids(7, 2048, cfg.vocab_size)
    kv = model.new_cache(1, 2048 + 32)
    model.try_forward_cached_last(prompt[:8], kv)  # staging buffers, scratch
    kv.reset(0)
    t0 = time.perf_counter()
    model.try_forward_cached_last(prompt, kv)
    t_pre = time.perf_counter() - t0
    n_dec = 4
    t0 = time.perf_counter()
    for i in range(n_dec):
        model.try_forward_cached_last([i + 1], kv)
    t_dec = (time.perf_counter() - t0) / n_dec
    reads = model.streaming_stats().layer_reads
    link = h2d_gbs()
    # every layer kept in HBM after one pass; greedy generation then replays
    # the captured decode step (difference of 40- and 8-token loops over the
    # same prompt, so the prefill cancels)
    model.with_layer_cache(1 << 40)
    kv.reset(0)
    model.try_forward_cached_last(prompt, kv)

    dev = {}

    def gen(n):
        t0 = time.perf_counter()
        out = model.generate_greedy_device(model.new_cache(1, 2048 + 48), prompt, n, eos=[])
        assert len(out) == n
        dev["ids"] = out
        return time.perf_counter() - t0

    gen(8)
    t_cached = (gen(40) - gen(8)) / 32
    dc = model.streaming_stats().device_cache
    greedy_self_check(model, kv, prompt, dev["ids"])
    res = {"workload": "C3 shape (Llama-3-8B, bf16, no LoRA), every layer streamed from host "
                       "safetensors artifacts per forward; 2048-token prefill, batch-1 decode at "
                       "2048+ context; then a device layer cache holding all 32 layers (greedy "
                       "device loop)",
           "streamed_bytes_per_forward": per_forward,
           "streamed_prefill_2048_ms": round(t_pre * 1e3, 2),
           "streamed_decode_ms_per_token": round(t_dec * 1e3, 2),
           "streamed_gbs": round(per_forward / t_dec / 1e9, 2),
           "h2d_pinned_gbs": round(link, 2),
           "streamed_link_frac": round(per_forward / t_dec / 1e9 / link, 4),
           "layer_reads": reads,
           "cached_decode_ms_per_token": round(t_cached * 1e3, 3),
           "cached_layers": dc.layers, "cache_hits": dc.hits}
    model.close()
    return res


def c4_config(max_pos=4096):
    from esp_amd.config import DecoderConfig
    return DecoderConfig.mixtral_style(vocab_size=32000, hidden_size=4096, intermediate_size=14336,
                                       num_hidden_layers=4, num_attention_heads=32,
                                       num_key_value_heads=8, max_position_embeddings=max_pos,
                                       rope_theta=1000000.0, num_experts=8, num_experts_per_tok=2,
                                       moe_intermediate_size=14336)


def moe_decode_bytes(cfg, ctx: int) -> int:
    """Algorithmic HBM bytes of one batch-1 MoE decode step: attention
    weights, router and the top-k experts' gate/up/down rows of every layer
    (bf16), the head (bf16) and the K/V cache once (2 bytes per element, as
    BASELINE.md counts it)."""
    H, L, V = cfg.hidden_size, cfg.num_hidden_layers, cfg.vocab_size
    qw, kvw = cfg.query_width(), cfg.kv_heads() * cfg.head_dim()
    m = cfg.moe
    layer = (H * (qw + 2 * kvw) + H * qw + m.num_experts * H
             + m.num_experts_per_tok * 3 * H * m.moe_intermediate_size) * 2
    return L * layer + V * H * 2 + 2 * L * kvw * ctx * 2


def moe_prefill_flops(cfg, S: int) -> float:
    """Useful FLOPs of an S-token MoE prefill: projections, router, the top-k
    experts each token is routed to, causal attention, last-position head."""
    H, L, V = cfg.hidden_size, cfg.num_hidden_layers, cfg.vocab_size
    qw, kvw, hd, nq = cfg.query_width(), cfg.kv_heads() * cfg.head_dim(), cfg.head_dim(), \
        cfg.num_attention_heads
    m = cfg.moe
    per_tok = H * (qw + 2 * kvw) + H * qw + m.num_experts * H + \
        m.num_experts_per_tok * 3 * H * m.moe_intermediate_size
    return 2.0 * S * L * per_tok + 2.0 * 2.0 * L * nq * hd * S * (S + 1) / 2 + 2.0 * H * V


def c4_bench(steps: int) -> dict:
    """Mixtral-style MoE stack (4 layers, hidden 4096,
    8 experts of SwiGLU 14336, top-2 softmax router, vocab 32000), bf16,
    synthetic N(0, 0.02) weights: a 2048-token uniform-random prefill, then
    batch-1 greedy decode at ~2048 context (device loop, captured step)."""
    from esp_amd import DecoderModel
    cfg = c4_config()
    model = DecoderModel.synthetic(cfg, seed=777, std=0.02, fmt="bf16")
    prompt = uniform_ids(17, 2048, cfg.vocab_size)
    n_dec = 64
    kv = model.new_cache(1, 2048 + n_dec)

    def prefill():
        kv.reset(0)
        t0 = time.perf_counter()
        model.try_forward_cached_last(prompt, kv)
        return time.perf_counter() - t0

    dev = {}

    def gen():
        t0 = time.perf_counter()
        out = model.generate_greedy_device(kv, prompt, n_dec, eos=[])
        assert len(out) == n_dec
        dev["ids"] = out
        return time.perf_counter() - t0

    gen()
    prefill()
    t_gen = sorted(gen() for _ in range(steps))[steps // 2]
    t_pre = sorted(prefill() for _ in range(steps))[steps // 2]
    greedy_self_check(model, kv, prompt, dev["ids"])
    t_dec = (t_gen - t_pre) / (n_dec - 1)
    db = moe_decode_bytes(cfg, 2048 + n_dec // 2)
    fl = moe_prefill_flops(cfg, 2048)
    res = {"workload": "C4: Mixtral-style MoE (4 layers, hidden 4096, 8 experts x SwiGLU 14336, "
                       "top-2), bf16; 2048-token prefill, batch-1 decode at 2048-2112 context "
                       "(BASELINE configs[3])",
           "decode_tokens_per_s": round(1.0 / t_dec, 2),
           "decode_ms_per_token": round(t_dec * 1e3, 4),
           "decode_hbm_frac": round(db / t_dec / 1e9 / HBM_PEAK_GBS, 4),
           "decode_bytes_per_token": db,
           "prefill_2048_tokens_per_s": round(2048 / t_pre, 1),
           "prefill_2048_ms": round(t_pre * 1e3, 3),
           "prefill_mfma_frac": round(fl / t_pre / 1e12 / BF16_PEAK_TFLOPS, 4)}
    model.close()
    return res


def c5_bench(steps: int, warmup: int = 2, kv_dtype: str = "f32") -> dict:
    """constrained decode on the 1B shape, 64 concurrent
    sequences at ~1024 context. Each step: every sequence whose index is
    congruent to the step mod 8 evaluates a forced 8-token block (a causal
    mini-prefill over its warm cache), the other 56 one decode token; then
    one esp_pick over the 64 last-position logits rows applies a
    per-sequence allowed-token bitmask (Bernoulli 0.05 from the seed, at
    least one token allowed) and seeded temperature 0.8 / top-p 0.9
    sampling (sample.rs:83-121). Sequences are prefilled with 1024
    uniform-random ids before timing."""
    import numpy as np
    from esp_amd import DecoderModel, Sampler
    cfg = c2_config(max_pos=2048)
    B, ctx0, V = 64, 1024, cfg.vocab_size
    total = warmup + steps
    model = DecoderModel.synthetic(cfg, seed=1234, std=0.02, fmt="bf16")
    kv = model.new_cache(B, ctx0 + 8 * total + 8, kv_dtype)
    model.forward_batch(kv, list(range(B)), [uniform_ids(5000 + i, ctx0, V) for i in range(B)],
                        want_logits=False)
    words = (V + 31) // 32
    rng = np.random.default_rng(20261201)
    masks = []
    for st in range(total):
        allow = rng.random((B, words * 32), dtype=np.float32) < 0.05
        allow[:, V:] = False
        allow[np.arange(B), rng.integers(0, V, B)] = True  # at least one allowed
        masks.append(np.packbits(allow, axis=1, bitorder="little").view(np.uint32).copy())
    forced = [[uniform_ids(9000 + 100 * st + i, 8, V) for i in range(B)] for st in range(total)]
    samplers = [Sampler(0.8, 0.9, 0xC5C5 + i) for i in range(B)]
    last = [int(x) for x in rng.integers(0, V, B)]
    seqs = list(range(B))
    rows = 0

    def step(st):
        nonlocal rows
        blocks = []
        for i in range(B):
            if (i + st) % 8 == 0:
                blocks.append(forced[st][i])
                samplers[i].skip_draws(8)  # forced tokens consume one draw each
            else:
                blocks.append([last[i]])
        rows += sum(len(b) for b in blocks)
        model.forward_batch(kv, seqs, blocks, want_logits=False)
        ids, flags = model.pick(kv, B, masks[st], samplers)
        last[:] = ids.tolist()
        picked.append(ids)

    picked = []
    for st in range(warmup):
        step(st)
    rows = 0
    t0 = time.perf_counter()
    for st in range(warmup, total):
        step(st)
    el = time.perf_counter() - t0
    # every pick is a token its row's mask allows
    for st, ids in enumerate(picked):
        ids = ids.astype(np.int64)
        ok = (masks[st][np.arange(B), ids >> 5] >> (ids & 31).astype(np.uint32)) & 1
        if not (ids < V).all() or not ok.all():
            raise RuntimeError(f"C5 step {st}: a picked id is outside its row's allowed mask")
    ctx_mid = ctx0 + 8 * total // 2
    qkv_kv = 2 * cfg.num_hidden_layers * cfg.kv_heads() * cfg.head_dim() * 2
    step_bytes = decode_bytes(cfg, 0)["gemv_weights"] + B * ctx_mid * qkv_kv + 2 * B * V * 4 + B * words * 4
    res = {"workload": "C5: 1B shape bf16, 64 sequences at 1024-1200 context; per step 56 decode "
                       "rows + 8 forced 8-token blocks, allowed-token bitmask (5%) + seeded "
                       "temperature 0.8 / top-p 0.9 sampling (BASELINE configs[4])",
           "sequence_tokens_per_s": round(B * steps / el, 1),
           "rows_per_s": round(rows / el, 1),
           "ms_per_step": round(el / steps * 1e3, 3),
           "step_hbm_frac": round(step_bytes / (el / steps) / 1e9 / HBM_PEAK_GBS, 4),
           "step_bytes": step_bytes,
           "kv_dtype": kv_dtype,
           "steps": steps}
    model.close()
    return res


class _ByteIds:
    """Tokenises text as one id per byte: ids 0..255 of the synthetic
    128256-entry table are the single bytes, so forced spans round-trip."""

    class _Enc:
        def __init__(self, ids):
            self.ids = ids

    def encode(self, text, add_special_tokens=False):
        return self._Enc(list(text.encode("utf-8")))


def record_grammar():
    """A JSON record: five fields with bounded strings, a 16-way enum and a
    boolean (OutputGrammar serde form, provider.rs:55-75)."""
    def lit(v):
        return {"kind": "literal", "value": v}

    def string(n):
        return {"kind": "json_string", "max_bytes": n}
    kinds = {"kind": "choice", "alternatives": [lit(f"\"type_{i:02d}\"") for i in range(16)]}
    ok = {"kind": "choice", "alternatives": [lit("true"), lit("false")]}
    return {"kind": "sequence", "items": [
        lit("{\"id\":"), string(16), lit(",\"name\":"), string(48), lit(",\"kind\":"), kinds,
        lit(",\"ok\":"), ok, lit(",\"note\":"), string(96), lit("}")]}


def c5_grammar_bench(steps: int, warmup: int = 2) -> dict:
    """C5's batch with its allowed-token masks produced by real output
    grammars (provider.rs:735-883 run for 64 sequences at once): 1B shape
    bf16, 64 sequences prefilled with 1024 uniform-random ids, seeded
    temperature 0.8 / top-p 0.9. Each step, every sequence either takes its
    grammar's forced span (constraint.rs:296-344; the sampler skips one draw
    per forced token) or picks one token from its logits row masked on the
    device by its constraint (esp_pick_constrained); tokens are accepted into
    the constraints and all 64 blocks are evaluated by one forward. A
    sequence whose record completes starts the next record. The token table
    is a seeded synthetic 128256-entry byte-level vocabulary."""
    import numpy as np
    from esp_amd import DecoderModel, Sampler
    from esp_amd.constraint import Constraint, Vocabulary
    from esp_amd.model import profile_enable, profile_read
    cfg = c2_config(max_pos=4096)
    B, ctx0, V = 64, 1024, cfg.vocab_size
    total = warmup + steps
    vocab = Vocabulary(llama_sized_table(n=V))
    tok = _ByteIds()
    grammar = json.dumps(record_grammar())
    model = DecoderModel.synthetic(cfg, seed=1234, std=0.02, fmt="bf16")
    kv = model.new_cache(B, ctx0 + 64 * total + 64)
    model.forward_batch(kv, list(range(B)), [uniform_ids(5000 + i, ctx0, V) for i in range(B)],
                        want_logits=False)
    cons = [Constraint(grammar, vocab=vocab) for _ in range(B)]
    samplers = [Sampler(0.8, 0.9, 0xC5C5 + i) for i in range(B)]
    seqs = list(range(B))
    stats = {"tokens": 0, "forced": 0, "picked": 0, "records": 0}
    t_mask = [0.0]

    def step():
        blocks, rows_c, rows_s = [], [], []
        for i in range(B):
            f = cons[i].forced(tok)
            blocks.append(f)
            rows_c.append(None if f else cons[i])
            rows_s.append(None if f else samplers[i])
            if f:
                samplers[i].skip_draws(len(f))
        ids, _ = model.pick_constrained(kv, rows_c, rows_s)
        for i in range(B):
            if blocks[i]:
                stats["forced"] += len(blocks[i])
            else:
                blocks[i] = [int(ids[i])]
                stats["picked"] += 1
            for t in blocks[i]:
                cons[i].accept(t)
            stats["tokens"] += len(blocks[i])
            if cons[i].complete():
                stats["records"] += 1
                cons[i] = Constraint(grammar, vocab=vocab)
        model.forward_batch(kv, seqs, blocks, want_logits=False)

    # a first forward so every row holds logits before the first pick
    model.forward_batch(kv, seqs, [[1]] * B, want_logits=False)
    for _ in range(warmup):
        step()
    for k in stats:
        stats[k] = 0
    profile_enable("cmask", True)
    m0 = profile_read("cmask")
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    el = time.perf_counter() - t0
    m1 = profile_read("cmask")
    profile_enable("cmask", False)
    res = {"workload": "C5 with grammar masks: 1B shape bf16, 64 sequences from 1024 context, "
                       "JSON-record output grammar per sequence, device masks + forced spans, "
                       "seeded temperature 0.8 / top-p 0.9; synthetic 128256-entry byte-level "
                       "token table",
           "sequence_tokens_per_s": round(stats["tokens"] / el, 1),
           "steps_per_s": round(steps / el, 2),
           "ms_per_step": round(el / steps * 1e3, 3),
           "mask_ms_per_step": round((m1[1] - m0[1]) / max(1, m1[0] - m0[0]), 4),
           "forced_tokens": stats["forced"], "picked_tokens": stats["picked"],
           "records_completed": stats["records"], "steps": steps}
    model.close()
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--no-cpu", action="store_true")
    for leg in ("c2", "c4", "c5", "c5g", "packed", "stream"):
        ap.add_argument(f"--no-{leg}", action="store_true")
        ap.add_argument(f"--only-{leg}", action="store_true")
    ap.add_argument("--only-c3", action="store_true", help="the headline leg alone (no CPU baseline)")
    ap.add_argument("--traffic", action="store_true",
                    help="run only the workload of the HBM-traffic counter passes")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(multi-GPU sharding is design-only)"}))
        sys.exit(2)
    steps = max(1, args.steps)
    if args.traffic:
        traffic_run()
        return
    only = {"c2": lambda: c2_bench(steps, args.warmup), "c4": lambda: c4_bench(steps),
            "c5": lambda: {d: c5_bench(16, kv_dtype=d) for d in ("f32", "f16")},
            "c5g": lambda: c5_grammar_bench(32),
            "stream": lambda: c3_stream_bench()}
    for leg, fn in only.items():
        if getattr(args, f"only_{leg}"):
            print(json.dumps({leg: fn()}), flush=True)
            return
    if args.only_c3:
        print(json.dumps({"c3": c3_headline(steps, args.warmup)}), flush=True)
        return
    if args.only_packed:
        print(json.dumps({"c3_q8": c3_packed_bench(8), "c3_q4": c3_packed_bench(4)}), flush=True)
        return
    cfg = c3_config()
    h = c3_headline(steps, args.warmup)
    result = {
        "metric": "decode & prefill tokens/s on 1 MI355X; % of HBM / bf16-MFMA roofline",
        "value": h["value"],
        "unit": "tokens/s (decode, batch 1)",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": h["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 weights, f32 activations/accumulation",
        "data": "synthetic (random-init N(0,0.02) weights, LoRA A~N(0,0.02) B~N(0,0.01), "
                "uniform-random prompt ids)",
        "config": {"workload": "C3: Llama-3-8B shape bf16 + LoRA r16 alpha 32 on q/v; 4064-token "
                               "prompt then 64 greedy decode steps (decode at 4064-4128 context), "
                               "batch 1; separate 2048-token prefill (BASELINE configs[2])",
                   "global_batch": 1, "seq_len": 4128, "parallelism": "none (1 GPU)"},
    }
    result.update({k: v for k, v in h.items() if k not in ("value", "ms_per_step")})
    print(f"c3: decode {h['value']} tok/s ({h['decode_hbm_frac']} of HBM on BASELINE bytes), "
          f"prefill {h['prefill_tokens_per_s']} tok/s", file=sys.stderr, flush=True)
    legs = [("c2", lambda: c2_bench(steps, args.warmup)), ("c4", lambda: c4_bench(steps)),
            ("c5", lambda: c5_bench(16)), ("c5_grammar", lambda: c5_grammar_bench(32))]
    for name, fn in legs:
        if not getattr(args, "no_" + ("c5g" if name == "c5_grammar" else name)):
            result[name] = fn()
            print(f"{name}: {result[name]}", file=sys.stderr, flush=True)
    if not args.no_packed:
        for bits in (8, 4):
            result[f"c3_q{bits}"] = c3_packed_bench(bits)
            print(f"c3_q{bits}: {result[f'c3_q{bits}']}", file=sys.stderr, flush=True)
    if not args.no_stream:
        result["c3_stream"] = c3_stream_bench()
        print(f"c3_stream: {result['c3_stream']}", file=sys.stderr, flush=True)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(cfg)
        print(f"cpu_baseline: {result['cpu_baseline']}", file=sys.stderr, flush=True)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
