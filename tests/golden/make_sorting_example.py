"""Writes moe_sorting_worked_example.json: the worked example of the
reference's sorting kernel, transcribed from the comment in
csrc/include/moe_sorting_opus.h:277-339 (no reference code is run).

The comment lists, per expert, the token ids and the weights (letters a..o
for topk_weight read row-major); the encoded entries are
(slot << 24) | token with the slot found from topk_ids, and padding entries
are (topk << 24) | tokens with weight 0 (op_tests/test_moe_sorting.py:29).
Two slips of the comment are corrected: it prints padding tokens as 6 (the
closed form gives tokens = 5) and expert 5's last token as 5 (topk_ids put
expert 5 in token 4's top-k). The output is the variant that skips experts
without tokens, which is what aiter's moe_sorting produces (the second
listing of the comment).

    python tests/golden/make_sorting_example.py
"""
import json
from pathlib import Path

TOPK_IDS = [[0, 3, 5], [2, 3, 5], [1, 3, 5], [1, 2, 3], [1, 3, 5]]
LETTERS = "abcdefghijklmno"                     # topk_weight, row-major
WEIGHT = {ch: float(i + 1) for i, ch in enumerate(LETTERS)}
TOKENS, TOPK, E, BLOCK = 5, 3, 6, 4
# token_id_per_expert / weight_id_per_expert of the comment (expert 5: token 4)
PER_EXPERT = {0: ([0], "a"), 1: ([2, 3, 4], "gjm"), 2: ([1, 3], "dk"),
              3: ([0, 1, 2, 3, 4], "behln"), 4: ([], ""), 5: ([0, 1, 2, 4], "cfio")}


def layout(mask):
    ids, ws, eids = [], [], []
    local = 0
    for e in range(E):
        toks, letters = PER_EXPERT[e]
        if mask[e] and toks:
            for t, ch in zip(toks, letters):
                slot = TOPK_IDS[t].index(e)
                ids.append((slot << 24) | t)
                ws.append(WEIGHT[ch])
            pad = -len(toks) % BLOCK
            ids += [(TOPK << 24) | TOKENS] * pad
            ws += [0.0] * pad
            eids += [local] * ((len(toks) + pad) // BLOCK)
        local += mask[e]
    return {"sorted_token_ids": ids, "sorted_weights": ws, "sorted_expert_ids": eids,
            "num_valid_ids": [len(ids), TOKENS]}


def fixture():
    return {
        "source": "csrc/include/moe_sorting_opus.h:277-339 (see make_sorting_example.py)",
        "num_experts": E, "topk": TOPK, "block_size": BLOCK, "tokens": TOKENS,
        "topk_ids": TOPK_IDS,
        "topk_weights": [[WEIGHT[LETTERS[3 * t + j]] for j in range(TOPK)]
                         for t in range(TOKENS)],
        "unmasked": layout([1] * E),
        "masked": dict(layout([1, 0, 1, 1, 0, 1]), expert_mask=[1, 0, 1, 1, 0, 1]),
    }


OUT = Path(__file__).with_name("moe_sorting_worked_example.json")

if __name__ == "__main__":
    OUT.write_text(json.dumps(fixture(), indent=1) + "\n")
    print(f"wrote {OUT}")
