"""Write tests/golden/known_answers.json: hand-derived vectors for the oracle pins.

Nothing here calls the oracle or the reference. Every expected value follows
from a closed form stated next to it:
  * attention with q = 0 averages the visible V rows;
  * two keys whose scores differ by ln 3 get weights 3/4 and 1/4;
  * a causal query that sees only key 0 returns V row 0;
  * int4 words from the bit layout "nibble n of word j = q[8j + n] at bits 4n"
    (slipstream/kernels/quant_ref.py:18-19), the vectors of the reference's own
    tests/correctness/test_quant_w4a16.py:38-42;
  * dequantisation (q - zero) * scale with exactly representable numbers.
Run: python tests/golden/make_known_answers.py
"""

from __future__ import annotations

import json
import math
from pathlib import Path


def attention_cases() -> list[dict]:
    cases = []
    # 1. q = 0: every visible key has the same score -> mean of V. Pool of 3 blocks (bs 2),
    #    sequence of 3 tokens through table [2, 0]; n_q 2 / n_kv 1 (GQA).
    bs, nb, d = 2, 3, 2
    kv = [[[[[[0.0] * d] for _ in range(bs)] for _ in range(nb)] for _ in range(2)]]
    vals = {0: [1.0, 2.0], 1: [3.0, 6.0], 2: [5.0, -4.0]}  # V of tokens 0..2
    table = [2, 0]
    for t, vec in vals.items():
        blk, off = table[t // bs], t % bs
        kv[0][1][blk][off][0] = vec
        kv[0][0][blk][off][0] = [float(t), 1.0]  # K arbitrary: q = 0 ignores it
    mean = [sum(vals[t][x] for t in range(3)) / 3 for x in range(d)]
    cases.append({"name": "q0_mean_of_values", "block_size": bs, "scale": 0.125,
                  "q": [[[[0.0, 0.0]], [[0.0, 0.0]]]], "kv_cache": kv, "block_tables": [table],
                  "seq_lens": [3], "expected": [[[mean, mean]]]})
    # 2. two keys with scores ln 3 and 0 -> weights 3/4, 1/4 (scale 1, n_q = n_kv = 1).
    bs, nb, d = 4, 1, 2
    kv = [[[[[[0.0] * d] for _ in range(bs)] for _ in range(nb)] for _ in range(2)]]
    kv[0][0][0][0][0] = [math.log(3.0), 0.0]
    kv[0][0][0][1][0] = [0.0, 0.0]
    kv[0][1][0][0][0] = [4.0, 8.0]
    kv[0][1][0][1][0] = [0.0, -4.0]
    cases.append({"name": "two_keys_ln3", "block_size": bs, "scale": 1.0,
                  "q": [[[[1.0, 0.0]]]], "kv_cache": kv, "block_tables": [[0]], "seq_lens": [2],
                  "expected": [[[[3.0, 5.0]]]]})
    # 3. Tq = 2 over 2 keys: query 0 sits at position 0 and sees only key 0 -> V0;
    #    query 1 sees both with scores ln3, 0 -> 3/4 V0 + 1/4 V1.
    cases.append({"name": "causal_chunk_offset", "block_size": bs, "scale": 1.0,
                  "q": [[[[1.0, 0.0], [1.0, 0.0]]]], "kv_cache": kv, "block_tables": [[0]], "seq_lens": [2],
                  "expected": [[[[4.0, 8.0]], [[3.0, 5.0]]]]})
    return cases


def int4_cases() -> dict:
    def word(nibbles):
        w = 0
        for n, q in enumerate(nibbles):
            w |= (q & 0xF) << (4 * n)
        return w - (1 << 32) if w >= (1 << 31) else w

    rows = [[15] * 8, [0, 1, 2, 3, 12, 13, 14, 15], [1, 0, 0, 0, 0, 0, 0, 8]]
    return {
        "nibbles": rows,
        "packed": [[word(r)] for r in rows],  # -1, 0xFEDC3210 as int32, 0x80000001 as int32
        "dequant": {
            "q": [[0, 8, 15, 9, 1, 2, 3, 4]],
            "zero": [[8]],
            "scale": [[0.5]],
            "group_size": 8,
            "expected": [[(q - 8) * 0.5 for q in [0, 8, 15, 9, 1, 2, 3, 4]]],
        },
    }


def main() -> None:
    out = {"attention": attention_cases(), "int4": int4_cases()}
    path = Path(__file__).resolve().parent / "known_answers.json"
    path.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
