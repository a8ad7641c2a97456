"""Writes tests/golden/gguf_kat.json: the GGUF block known-answer vectors of the
reference's own test (tests/test_advanced_experiments.py:85-92 and 116-121),
as raw block bytes plus the expected fp32 values stated there in closed form:

* Q8_0: d = fp16(0.5), q = arange(-16, 16)        -> q * 0.5
* Q4_0: d = fp16(0.25), low nibbles = arange(16), high nibbles = 15 - arange(16)
        -> elements 0..15 = (low - 8) * 0.25, 16..31 = (high - 8) * 0.25

The expected values are computed here from those closed forms, not by any decoder.
Run: python tests/golden/make_golden.py
"""
import json
from pathlib import Path

import numpy as np

q8_values = np.arange(-16, 16, dtype=np.int8)
q8_block = np.float16(0.5).tobytes() + q8_values.tobytes()
q8_expected = [float(v) * 0.5 for v in q8_values.tolist()]

low = np.arange(16, dtype=np.uint8) & 0x0F
high = (15 - np.arange(16, dtype=np.uint8)) & 0x0F
q4_block = np.float16(0.25).tobytes() + (low | (high << 4)).astype(np.uint8).tobytes()
q4_expected = [(int(v) - 8) * 0.25 for v in low.tolist()] + [(int(v) - 8) * 0.25 for v in high.tolist()]

out = {
    "source": "tests/test_advanced_experiments.py:85-92,116-121 (reference)",
    "q8_0": {"block_hex": q8_block.hex(), "expected": q8_expected},
    "q4_0": {"block_hex": q4_block.hex(), "expected": q4_expected},
}
Path(__file__).with_name("gguf_kat.json").write_text(json.dumps(out, indent=1))
print("wrote gguf_kat.json")
