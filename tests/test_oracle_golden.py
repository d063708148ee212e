"""The CPU oracle against the reference's committed Transformers goldens
(crates/esp/tests/support/architectures/reference.json; checked the way
architecture_tests.rs:237-262 checks esp: last logits < 2e-5, 4 greedy ids
exact)."""
import hashlib
import json
import os

import numpy as np
import pytest

from esp_amd.config import DecoderConfig
from oracle import oracle, st

ARCH = os.path.join(os.path.dirname(__file__), "golden", "arch")
REF = json.load(open(os.path.join(ARCH, "reference.json")))


@pytest.mark.parametrize("case", [c["name"] for c in REF["cases"]])
def test_oracle_matches_transformers_golden(case):
    row = next(c for c in REF["cases"] if c["name"] == case)
    blob = open(os.path.join(ARCH, case, "model.safetensors"), "rb").read()
    assert hashlib.sha256(blob).hexdigest() == row["weights_sha256"]
    cfg = DecoderConfig.from_json_bytes(open(os.path.join(ARCH, case, "config.json"), "rb").read())
    m = oracle.OracleModel(cfg, st.load(blob))
    kv = m.new_cache()
    logits = m.forward_last(kv, row["input_ids"])
    assert np.abs(logits - np.array(row["last_logits"], np.float32)).max() < 2e-5
    gen = []
    for step in range(4):
        if step:
            logits = m.forward_last(kv, [gen[-1]])
        gen.append(oracle.argmax(logits))
    assert gen == row["generated_ids"]
