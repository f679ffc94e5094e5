"""Write tests/golden/gemma2b_greedy.json: the C oracle's greedy run of the
Gemma-2B-shaped model (18 layers, hidden 2048, 8 Q / 1 KV heads of dim 256,
GeGLU 16384, vocab 256000, eps 1e-6, RoPE base 10000) with synthetic
N(0, 0.02^2) weights (hash generator, seed SEED), a prompt of 128 uniform-random
token ids, then 256 greedy tokens.

    python tests/golden/make_gemma2b_greedy.py        # ~2 minutes on 8 cores

Besides the tokens it records, per generated token, the top-1 minus top-2 logit
margin, and at a few positions the top-16 logits and the logits' sum and sum of
squares, so the GPU run can be compared on values as well as on token ids.
"""

from __future__ import annotations

import json
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import model as om, native  # noqa: E402

OUT = Path(__file__).resolve().parent / "gemma2b_greedy.json"
SEED = 1234
PROMPT_LEN = 128
N_NEW = 256
MAX_CTX = 384
PROBE_POS = (PROMPT_LEN - 1, 200, PROMPT_LEN + N_NEW - 2)


def prompt_ids(seed: int = SEED) -> list[int]:
    return np.random.default_rng(seed).integers(0, om.GEMMA_2B.vocab, PROMPT_LEN).astype(np.int64).tolist()


def main() -> None:
    t0 = time.time()
    dec = native.NativeDecoder(om.GEMMA_2B, MAX_CTX, SEED)
    print(f"weights generated in {time.time() - t0:.1f} s", flush=True)
    prompt = prompt_ids()
    dec.tokens[:PROMPT_LEN] = prompt
    margins, probes = [], {}
    for pos in range(PROMPT_LEN + N_NEW - 1):
        want = pos in PROBE_POS
        _, m, logits = dec.step(pos, want_logits=want, sample=pos >= PROMPT_LEN - 1)
        if pos >= PROMPT_LEN - 1:
            margins.append(m)
        if want:
            top = np.argsort(-logits, kind="stable")[:16]
            probes[str(pos)] = {
                "top_ids": top.tolist(),
                "top_logits": logits[top].astype(float).tolist(),
                "sum": float(logits.astype(np.float64).sum()),
                "sumsq": float((logits.astype(np.float64) ** 2).sum()),
            }
        if pos % 32 == 0:
            print(f"pos {pos} {time.time() - t0:.0f} s", flush=True)
    tokens = [int(t) for t in dec.tokens[PROMPT_LEN : PROMPT_LEN + N_NEW]]
    json.dump({"seed": SEED, "std": 0.02, "max_ctx": MAX_CTX, "prompt": prompt, "tokens": tokens,
               "margins": margins, "probes": probes}, OUT.open("w"))
    print(f"wrote {OUT}: {len(set(tokens))} distinct tokens, min margin {min(margins):.4f}")


if __name__ == "__main__":
    main()
