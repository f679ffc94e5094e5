"""The drop-in surface end to end on the GPU: a local HF-layout Gemma checkpoint
is converted to the reference's flat weight file, loaded by the engine binary
(run as a subprocess, the way KernelRunner, ios_kernels/surfaces/runners/
kernel_runner.py:29-44, and the benchmark harness, ios_kernels/benchmarking/
bench.py:45-61, start it) and must reproduce HF transformers' greedy tokens and
logits for that checkpoint (tests/golden/hf_gemma_tiny.npz).

Tolerances: token ids identical. Logits, max|got - ref| / max|ref| against HF
in float64: <= 1e-3 through the token-by-token prefill (fp16 weights, fp32
activations and accumulation), and the 1e-2 contract through the batched
prefill, which rounds its activation rows to fp16 where the reference's prefill
chunk does (xnHalf / attHalf / hidHalf, KL/main.swift:412-446).
"""

from __future__ import annotations

import json
import os
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from oracle import model as om
from tests.conftest import rel_err
from tests.test_weights_serve import _hf_snapshot

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = np.load(Path(__file__).resolve().parent / "golden" / "hf_gemma_tiny.npz")
PROMPT = [int(t) for t in GOLDEN["prompt"]]
GREEDY = [int(t) for t in GOLDEN["greedy"]]


@pytest.fixture(scope="module")
def weights_file(tmp_path_factory):
    from gemmagemini4hackathon2026_10_2425_amd import weights

    d = tmp_path_factory.mktemp("hf")
    _hf_snapshot(d / "snap", om.TINY, int(GOLDEN["seed"]), std=float(GOLDEN["std"]),
                 embed_std=float(GOLDEN["embed_std"]))
    weights.convert_hf(d / "snap", d / "gemma_tiny.bin")
    return d / "gemma_tiny.bin"


def _run(args, stdin: str = "", timeout: int = 240):
    """The engine binary as a child process; (returncode, stdout, stderr)."""
    p = subprocess.run([sys.executable, "-m", "gemmagemini4hackathon2026_10_2425_amd.serve", *map(str, args)],
                       input=stdin, capture_output=True, text=True, timeout=timeout, cwd=ROOT, env=dict(os.environ))
    return p.returncode, p.stdout, p.stderr


def test_load_engine_matches_hf(dev, weights_file):
    """In process: the loaded engine's greedy tokens equal HF's."""
    from gemmagemini4hackathon2026_10_2425_amd.weights import load_engine

    from gemmagemini4hackathon2026_10_2425_amd import _lib

    with load_engine(weights_file, 64) as e:
        assert e.generate(PROMPT, len(GREEDY)) == GREEDY
        e.set_tokens(PROMPT)
        e.prefill(len(PROMPT))
        assert rel_err(e.logits(), GOLDEN["logits"][-1]) <= 1e-2
        _lib.set_tunable("ENG_NO_GEMM", 1)
        try:
            e.set_tokens(PROMPT)
            e.prefill(len(PROMPT))
        finally:
            _lib.set_tunable("ENG_NO_GEMM", 0)
        assert rel_err(e.logits(), GOLDEN["logits"][-1]) <= 1e-3


def test_serve_protocol_matches_hf(dev, weights_file):
    stop = GREEDY[2]
    k = GREEDY.index(stop)  # tokens before the first occurrence of the stop id
    reqs = [
        {"ids": PROMPT, "max_tokens": len(GREEDY)},
        {"ids": PROMPT, "max_tokens": len(GREEDY), "stop_ids": [stop]},
        {"ids": [10**6]},
        {"ids": PROMPT, "max_tokens": 3},
    ]
    rc, out, err = _run(["--weights", weights_file, "--serve", "--max-ctx", 64],
                        "".join(json.dumps(r) + "\n" for r in reqs))
    assert rc == 0, err[-2000:]
    msgs = [json.loads(l) for l in out.splitlines()]
    ready = msgs.pop(0)
    assert ready["ready"] is True and ready["max_ctx"] == 64 and ready["vocab"] == om.TINY.vocab
    assert isinstance(ready["device"], str) and ready["device"]

    def take():
        toks = []
        while "token" in msgs[0]:
            toks.append(msgs.pop(0)["token"])
        return toks, msgs.pop(0)

    toks, done = take()
    assert toks == GREEDY
    assert done == {**done, "done": True, "finish_reason": "length", "prompt_tokens": len(PROMPT),
                    "completion_tokens": len(GREEDY)}
    toks, done = take()
    assert toks == GREEDY[:k] and done["finish_reason"] == "stop" and done["completion_tokens"] == k
    assert msgs.pop(0) == {"error": f"token id {10**6} out of range"}
    toks, done = take()  # the server kept running after the bad request
    assert toks == GREEDY[:3] and done["finish_reason"] == "length"
    assert msgs == []
    assert "device:" in err


def test_cli_generate_and_dump_logits(dev, weights_file, tmp_path):
    rc, out, err = _run(["--weights", weights_file, "--max-ctx", 64, "--prompt-ids", ",".join(map(str, PROMPT)),
                         "--gen", len(GREEDY), "--dump-logits", tmp_path / "logits.f32"])
    assert rc == 0, err[-2000:]
    r = json.loads(out.strip().splitlines()[-1])
    assert r["tokens"] == GREEDY and r["decode_tok_s"] > 0
    logits = np.fromfile(tmp_path / "logits.f32", "<f4")
    assert logits.shape == (om.TINY.vocab,) and rel_err(logits, GOLDEN["logits"][-1]) <= 1e-2
    rc, out, err = _run(["--weights", weights_file, "--max-ctx", 64, "--prompt-ids", ",".join(map(str, PROMPT)),
                         "--gen", len(GREEDY), "--dump-logits", tmp_path / "logits_nogemm.f32", "--no-gemm"])
    assert rc == 0, err[-2000:]
    assert json.loads(out.strip().splitlines()[-1])["tokens"] == GREEDY
    logits = np.fromfile(tmp_path / "logits_nogemm.f32", "<f4")
    assert rel_err(logits, GOLDEN["logits"][-1]) <= 1e-3


def test_cli_bench_lines(dev, weights_file):
    """--bench-pp / --bench-tg print the lines the benchmark harness greps
    (r"^(pp|tg)") and one JSON report."""
    rc, out, err = _run(["--weights", weights_file, "--max-ctx", 64, "--bench-pp", 16, "--bench-tg", 32, "--reps", 2,
                         "--define", "MV_NR=2"])
    assert rc == 0, err[-2000:]
    rep = json.loads(out.strip().splitlines()[-1])
    assert rep["tunables"] == {"MV_NR": 2} and rep["pp"]["n"] == 16 and rep["tg"]["n"] == 32
    assert rep["pp"]["tok_s"] > 0 and rep["tg"]["tok_s"] > 0
    lines = [l for l in err.splitlines() if re.match(r"^(pp|tg)", l)]
    assert len(lines) == 2 and all(re.match(r"^(pp16|tg32): [\d.]+ ± [\d.]+ tok/s$", l) for l in lines)


def test_kernel_folder_binary(dev, weights_file):
    """The kernel folder's `llm` (what kernel.json names) runs the same engine."""
    llm = ROOT / "gemmagemini4hackathon2026_10_2425_amd" / "kernel" / "llm"
    p = subprocess.run([sys.executable, str(llm), "--weights", str(weights_file), "--max-ctx", "64", "--prompt-ids",
                        ",".join(map(str, PROMPT)), "--gen", "4"], capture_output=True, text=True, timeout=240, cwd=ROOT)
    assert p.returncode == 0, p.stderr[-2000:]
    assert json.loads(p.stdout.strip().splitlines()[-1])["tokens"] == GREEDY[:4]


def test_load_engine_rejects_mismatched_file(dev, tmp_path):
    from gemmagemini4hackathon2026_10_2425_amd import weights

    cfg = {"model_type": "gemma", "vocab_size": 1000, "hidden_size": 256, "intermediate_size": 512,
           "num_hidden_layers": 1, "num_attention_heads": 4, "num_key_value_heads": 1, "head_dim": 128}
    w = om.make_weights(om.DecodeConfig(1, 256, 4, 1, 128, 512, 1000), 1)
    w["l0.wup"] = w["l0.wup"][:-1]  # one row short
    weights.write_bin(tmp_path / "bad.bin", cfg, w)
    with pytest.raises(ValueError, match="l0.wup"):
        weights.load_engine(tmp_path / "bad.bin", 64)
    del w["l0.wup"]
    weights.write_bin(tmp_path / "miss.bin", cfg, w)
    with pytest.raises(ValueError, match="missing tensor l0.wup"):
        weights.load_engine(tmp_path / "miss.bin", 64)
    w2 = om.make_weights(om.DecodeConfig(1, 256, 4, 1, 128, 512, 1000), 1)
    w2["lm_head"] = w2["embed"]
    weights.write_bin(tmp_path / "head.bin", cfg, w2)
    with pytest.raises(ValueError, match="lm_head"):
        weights.load_engine(tmp_path / "head.bin", 64)
