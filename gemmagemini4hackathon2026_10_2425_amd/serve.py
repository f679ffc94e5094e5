"""The engine binary of the reference's kernel folder contract, on the MI355X
engine: greedy generation, llama-bench style throughput and the --serve
JSON-lines protocol, with the reference binary's flags and output formats
(KL/main.swift:1-74 options, :494-547 serve loop, :553-622 main).

    python -m gemmagemini4hackathon2026_10_2425_amd.serve --weights W.bin --prompt-ids 2,9906 --gen 32
    python -m gemmagemini4hackathon2026_10_2425_amd.serve --weights W.bin --bench-tg 128 --bench-pp 512 --reps 5
    python -m gemmagemini4hackathon2026_10_2425_amd.serve --weights W.bin --serve --max-ctx 4096

--serve protocol (stdout, one JSON object per line; logs go to stderr):
    out (once): {"ready": true, "max_ctx": N, "vocab": V, "device": "..."}
    in:         {"ids": [int], "max_tokens": N, "stop_ids": [int]}
    out:        {"token": id}   per generated token as soon as it is known (a stop token is not sent)
    out:        {"done": true, "finish_reason": "stop"|"length", "prompt_tokens": P,
                 "completion_tokens": n, "prefill_s": s, "decode_s": s}
    out:        {"error": "..."} for a bad request (the server keeps running)
Requests are sequential and each starts from position 0. EOF on stdin exits.

--define NAME=VALUE sets a kernel tunable (mxd_set_tunable), the counterpart
of the reference's Metal #defines. Prefill runs the prompt in chunks through
the matrix-core products; --no-gemm steps it token by token through the
decode path instead (the ENG_NO_GEMM tunable).
"""

from __future__ import annotations

import argparse
import json
import math
import sys
import time
from typing import IO, Iterable

BOS_BENCH = 128000  # the reference's bench-tg start token (KL/main.swift:589), taken modulo the vocabulary


def _write(out: IO[str], obj: dict) -> None:
    out.write(json.dumps(obj) + "\n")
    out.flush()


def _stats(xs: list[float]) -> tuple[float, float]:
    """Mean and sample standard deviation (KL/main.swift:549-553)."""
    m = sum(xs) / len(xs)
    v = sum((x - m) ** 2 for x in xs) / max(len(xs) - 1, 1)
    return m, math.sqrt(v)


class Server:
    """The --serve request loop over an engine (anything with set_tokens,
    prefill, token, decode_streaming and shape.vocab)."""

    def __init__(self, engine, max_ctx: int, out: IO[str], device: str = "HIP"):
        self.e, self.max_ctx, self.out, self.device = engine, max_ctx, out, device
        self.vocab = engine.shape.vocab

    def warmup(self) -> None:
        """Both paths once (first launches pay one-time costs), then ready."""
        ids = [BOS_BENCH % self.vocab] * 2
        self.e.set_tokens(ids)
        self.e.prefill(2)
        self.e.decode(2, 2)
        _write(self.out, {"ready": True, "max_ctx": self.max_ctx, "vocab": self.vocab, "device": self.device})

    def handle(self, line: str) -> None:
        try:
            req = json.loads(line)
        except ValueError:
            req = None
        ids = req.get("ids") if isinstance(req, dict) else None
        if not isinstance(ids, list) or not ids or not all(isinstance(t, int) and not isinstance(t, bool) for t in ids):
            _write(self.out, {"error": 'expected {"ids": [int, ...], "max_tokens": int}'})
            return
        bad = next((t for t in ids if t < 0 or t >= self.vocab), None)
        if bad is not None:
            _write(self.out, {"error": f"token id {bad} out of range"})
            return
        if len(ids) >= self.max_ctx:
            _write(self.out, {"error": f"prompt has {len(ids)} tokens, max_ctx is {self.max_ctx}"})
            return
        mt = req.get("max_tokens", 256)
        max_tokens = min(mt if isinstance(mt, int) and not isinstance(mt, bool) else 256, self.max_ctx - len(ids))
        stop = set(t for t in (req.get("stop_ids") or []) if isinstance(t, int))

        produced, finish = 0, "length"

        def emit(t: int) -> bool:
            nonlocal produced, finish
            if t in stop:
                finish = "stop"
                return False
            _write(self.out, {"token": int(t)})
            produced += 1
            return produced < max_tokens

        n = len(ids)
        self.e.set_tokens(ids)
        t0 = time.perf_counter()
        self.e.prefill(n)  # also samples the first token
        t_prefill = time.perf_counter() - t0
        t1 = time.perf_counter()
        if max_tokens > 0 and emit(self.e.token(n)) and max_tokens > 1:
            self.e.decode_streaming(n, max_tokens - 1, emit)
        _write(self.out, {"done": True, "finish_reason": finish, "prompt_tokens": n, "completion_tokens": produced,
                          "prefill_s": t_prefill, "decode_s": time.perf_counter() - t1})

    def run(self, lines: Iterable[str]) -> None:
        for line in lines:
            self.handle(line.rstrip("\n"))


def generate(engine, ids: list[int], gen: int, max_ctx: int, dump_logits: str | None = None) -> dict:
    """--prompt-ids / --gen / --dump-logits (KL/main.swift:563-586)."""
    if len(ids) + gen > max_ctx:
        raise ValueError(f"{len(ids)} prompt ids + {gen} new tokens exceed max_ctx {max_ctx}")
    engine.set_tokens(ids)
    t0 = time.perf_counter()
    engine.prefill(len(ids))
    t_prefill = time.perf_counter() - t0
    if dump_logits:
        engine.logits().astype("<f4").tofile(dump_logits)
    t1 = time.perf_counter()
    if gen > 1:
        engine.decode(len(ids), gen - 1)
    t_decode = time.perf_counter() - t1
    return {"tokens": engine.tokens(len(ids), gen) if gen > 0 else [], "prefill_s": t_prefill, "decode_s": t_decode,
            "decode_tok_s": (gen - 1) / t_decode if gen > 1 else 0}


def bench(engine, pp: int, tg: int, reps: int, tunables: dict, err: IO[str]) -> dict:
    """--bench-pp / --bench-tg / --reps, llama-bench style (KL/main.swift:588-619)."""
    vocab = engine.shape.vocab
    report: dict = {"tunables": tunables}
    if pp > 0:
        engine.set_tokens([(i * 7919 % 100000 + 1000) % vocab for i in range(pp)])
        engine.prefill(pp)  # warm-up
        rates = []
        for _ in range(reps):
            t0 = time.perf_counter()
            engine.prefill(pp)
            rates.append(pp / (time.perf_counter() - t0))
        m, s = _stats(rates)
        report["pp"] = {"n": pp, "tok_s": m, "std": s}
        err.write(f"pp{pp}: {m:.1f} ± {s:.1f} tok/s\n")
    if tg > 0:
        bos = BOS_BENCH % vocab
        engine.set_tokens([bos])
        engine.decode(0, min(16, tg))  # warm-up
        rates = []
        for _ in range(reps):
            engine.set_tokens([bos])
            t0 = time.perf_counter()
            engine.decode(0, tg)
            rates.append(tg / (time.perf_counter() - t0))
        m, s = _stats(rates)
        report["tg"] = {"n": tg, "tok_s": m, "std": s}
        err.write(f"tg{tg}: {m:.1f} ± {s:.1f} tok/s\n")
    err.flush()
    return report


def parse_args(argv=None) -> argparse.Namespace:
    ap = argparse.ArgumentParser(prog="llm", description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--weights", required=True)
    ap.add_argument("--define", action="append", default=[], metavar="NAME=VALUE")
    ap.add_argument("--max-ctx", type=int, default=4096)
    ap.add_argument("--prompt-ids", default="")
    ap.add_argument("--gen", type=int, default=0)
    ap.add_argument("--bench-tg", type=int, default=0)
    ap.add_argument("--bench-pp", type=int, default=0)
    ap.add_argument("--reps", type=int, default=5)
    ap.add_argument("--dump-logits")
    ap.add_argument("--no-gemm", action="store_true")
    ap.add_argument("--serve", action="store_true")
    a = ap.parse_args(argv)
    a.tunables = {}
    for d in a.define:
        name, sep, val = d.partition("=")
        try:
            a.tunables[name] = int(val)
        except ValueError:
            sep = ""
        if not sep or not name:
            ap.error(f"--define {d!r}: expected NAME=INTEGER")
    try:
        a.ids = [int(t) for t in a.prompt_ids.split(",")] if a.prompt_ids else []
    except ValueError:
        ap.error(f"--prompt-ids {a.prompt_ids!r}: expected comma-separated integers")
    if a.max_ctx <= 0 or a.max_ctx % 32:
        ap.error(f"--max-ctx {a.max_ctx}: a positive multiple of 32")
    return a


def main(argv=None) -> int:
    a = parse_args(argv)
    from . import _lib
    from .weights import load_engine

    for name, val in a.tunables.items():
        _lib.set_tunable(name, val)
    if a.no_gemm:
        _lib.set_tunable("ENG_NO_GEMM", 1)
    try:
        import torch

        device = torch.cuda.get_device_name(0)
    except Exception:
        device = "HIP device"
    with load_engine(a.weights, a.max_ctx) as e:
        s = e.shape
        sys.stderr.write(f"device: {device}, dim {s.dim}, layers {s.n_layers}, vocab {s.vocab}, "
                         f"gemm {'false' if a.no_gemm else 'true'}\n")
        sys.stderr.flush()
        if a.ids:
            print(json.dumps(generate(e, a.ids, a.gen, a.max_ctx, a.dump_logits)), flush=True)
        if a.bench_pp > 0 or a.bench_tg > 0:
            if a.bench_pp + 1 > a.max_ctx or a.bench_tg + 1 > a.max_ctx:
                raise ValueError(f"bench sizes exceed max_ctx {a.max_ctx}")
            print(json.dumps(bench(e, a.bench_pp, a.bench_tg, a.reps, a.tunables, sys.stderr)), flush=True)
        if a.serve:
            srv = Server(e, a.max_ctx, sys.stdout, device)
            srv.warmup()
            srv.run(sys.stdin)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
