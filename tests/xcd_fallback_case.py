"""Child-process case of test_decode_attention_placement_fallback (run with
ESP_ATT_XCD_MISPLACE=1): every split-K decode-attention launch of the
XCD-local merge takes the linear block order, so a (row, kv head)'s splits
run on several XCDs. The launch's placement check must report it, and the
forward must then be computed again with the agent-scope merge: logits
within 1e-4 of the f32 oracle for a long prefill and four greedy steps,
and the device greedy loop equal to the host loop. A separate process,
because the fallback switches the XCD-local merge off for the process."""
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

from esp_amd import DecoderModel  # noqa: E402
from oracle import oracle, st  # noqa: E402
from tests import synth  # noqa: E402


# exit status when the device gives the XCD-local merge no placement to
# check (one XCD, or the dispatch-order probe failed): the test skips
NOT_APPLICABLE = 77


def main() -> int:
    assert os.environ.get("ESP_ATT_XCD_MISPLACE") == "1"
    from esp_amd.model import profile_read
    mode = profile_read("attn_xcd_mode")[0]
    print("attention merge mode", mode, flush=True)
    if mode <= 1:
        return NOT_APPLICABLE
    cfg = synth.llama_config(2, 256, 8, 2, 320, 300, head_dim=64, max_pos=1600)
    tensors = synth.make_tensors(cfg, 53, "f32")
    model = DecoderModel.from_bytes(cfg, st.dump(tensors), "f32")
    ref = oracle.OracleModel(cfg, tensors)
    prompt = synth.uniform_ids(6, 1500, cfg.vocab_size)
    # greedy device loop first: its first decode step meets the misplaced
    # launch inside the loop, which must then run again
    dev = model.generate_greedy_device(model.new_cache(1, 1540), prompt, 4, eos=[])
    kv, rkv = model.new_cache(1, 1540), ref.new_cache(1540)
    got = model.try_forward_cached_last(prompt, kv)
    want = ref.forward_last(rkv, prompt)
    ids = []
    for step in range(4):
        scale = float(np.abs(want).max())
        err = float(np.abs(got - want).max())
        print(f"step {step}: max |got - want| {err:.3g} (scale {scale:.3g})", flush=True)
        if err > 1e-4 * scale:
            return 1
        ids.append(int(np.argmax(got)))
        t = oracle.argmax(want)
        got = model.try_forward_cached_last([t], kv)
        want = ref.forward_last(rkv, [t])
    print("device loop", dev, "host loop", ids, flush=True)
    fallbacks = profile_read("attn_xcd_fallback")[0]
    print("placement fallbacks", fallbacks, flush=True)
    # the device loop's pass falls back once; afterwards the merge is off
    return 0 if dev == ids and fallbacks == 1 else 1


if __name__ == "__main__":
    sys.exit(main())
