"""Write the Gemma-2B-shaped greedy-run fixtures: the C oracle's greedy run of
the model (18 layers, hidden 2048, 8 Q / 1 KV heads of dim 256, GeGLU 16384,
vocab 256000, eps 1e-6, RoPE base 10000) with synthetic weights (hash
generator), a prompt of 128 uniform-random token ids, then 256 greedy tokens.

    python tests/golden/make_gemma2b_greedy.py            # both, ~2 minutes each on 8 cores

gemma2b_greedy.json
    every weight N(0, 0.02^2), the decode benchmark's model. Its greedy run is
    a fixed point: the sqrt(D)-scaled embedding of the current token dominates
    the residual stream, so the tied head picks that token again.
gemma2b_greedy_varied.json
    the same model with the embedding drawn N(0, 0.005^2), so the layers
    dominate the residual and the greedy tokens change at every step (the run
    that tells a correct engine from one that repeats its input).

Besides the tokens, each fixture records for every generated token the top-1
minus top-2 logit margin, the top-8 logits with their ids, and the logits' sum
and sum of squares, so the GPU run is compared on values at every step.
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

HERE = Path(__file__).resolve().parent
PROMPT_LEN = 128
N_NEW = 256
MAX_CTX = 384
TOP = 8
FIXTURES = {
    "gemma2b_greedy.json": dict(seed=1234, std=0.02, embed_std=0.02),
    "gemma2b_greedy_varied.json": dict(seed=1234, std=0.02, embed_std=0.005),
}


def prompt_ids(seed: int) -> list[int]:
    return np.random.default_rng(seed).integers(0, om.GEMMA_2B.vocab, PROMPT_LEN).astype(np.int64).tolist()


def write(name: str, seed: int, std: float, embed_std: float) -> None:
    t0 = time.time()
    dec = native.NativeDecoder(om.GEMMA_2B, MAX_CTX, seed, std, embed_std)
    prompt = prompt_ids(seed)
    dec.tokens[:PROMPT_LEN] = prompt
    margins, probes = [], []
    for pos in range(PROMPT_LEN + N_NEW - 1):
        sample = pos >= PROMPT_LEN - 1
        _, m, logits = dec.step(pos, want_logits=sample, sample=sample)
        if sample:
            margins.append(m)
            top = np.argsort(-logits, kind="stable")[:TOP]
            lg = logits.astype(np.float64)
            probes.append({"pos": pos, "top_ids": top.tolist(), "top_logits": logits[top].astype(float).tolist(),
                           "sum": float(lg.sum()), "sumsq": float((lg**2).sum())})
        if pos % 64 == 0:
            print(f"{name}: pos {pos} {time.time() - t0:.0f} s", flush=True)
    tokens = [int(t) for t in dec.tokens[PROMPT_LEN : PROMPT_LEN + N_NEW]]
    out = HERE / name
    json.dump({"seed": seed, "std": std, "embed_std": embed_std, "max_ctx": MAX_CTX, "prompt": prompt,
               "tokens": tokens, "margins": margins, "probes": probes}, out.open("w"))
    print(f"wrote {out}: {len(set(tokens))} distinct tokens, min margin {min(margins):.5f}")


def main() -> None:
    names = sys.argv[1:] or list(FIXTURES)
    for name in names:
        write(name, **FIXTURES[name])


if __name__ == "__main__":
    main()
