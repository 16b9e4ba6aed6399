"""End to end: the reference's own forward pass (slm_forward_batch prefill,
then greedy slm_forward_step decode) on a random Qwen3.5-0.8B-shaped
Q4_K_M model, once with its CPU matmuls (oracle/_ref/qwen_e2e_cpu) and
once with qk_seam.c routing every quantized matmul through libqk
(qwen.haiku_amd/host/_build/qwen_e2e_gpu). Both binaries are built from
the same driver (qwen.haiku_amd/host/qwen_e2e.c) and the same reference
sources with the same flags, so the greedy token streams must be
identical.
"""
import json
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
E2E_CPU = os.path.join(ROOT, "oracle", "_ref", "qwen_e2e_cpu")
E2E_GPU = os.path.join(ROOT, "qwen.haiku_amd", "host", "_build", "qwen_e2e_gpu")


def run(path, timeout, **kw):
    if not os.path.exists(path):
        pytest.fail(f"{path} is not built (make -C oracle; make -C qwen.haiku_amd/host)")
    args = [path]
    for k, v in kw.items():
        args += [f"--{k}", str(v)]
    print(f"[e2e] {' '.join(os.path.relpath(a, ROOT) if a == path else a for a in args)}", flush=True)
    r = subprocess.run(args, capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0, f"{path} failed ({r.returncode}):\n{r.stderr[-2000:]}"
    return json.loads(r.stdout.strip().splitlines()[-1])


def test_cpu_e2e_deterministic_and_nondegenerate():
    a = run(E2E_CPU, 120, prompt=8, gen=6, layers=4, seed=3)
    b = run(E2E_CPU, 120, prompt=8, gen=6, layers=4, seed=3)
    assert a["tokens"] == b["tokens"]
    assert a["nonfinite_logits"] == 0
    assert a["distinct_tokens"] >= 3
    assert a["last_logits"]["std"] > 0.1
    c = run(E2E_CPU, 120, prompt=8, gen=6, layers=4, seed=4)
    assert c["tokens"] != a["tokens"]


@pytest.mark.gpu
@pytest.mark.parametrize("prompt,gen", [(64, 16), (512, 256)])
def test_e2e_greedy_tokens_identical(prompt, gen):
    gpu = run(E2E_GPU, 240, prompt=prompt, gen=gen, seed=0)
    cpu = run(E2E_CPU, 240, prompt=prompt, gen=gen, seed=0)
    print(f"[e2e] gpu prefill {gpu['prefill_tok_s']:.1f} tok/s decode {gpu['decode_tok_s']:.1f} tok/s; "
          f"cpu prefill {cpu['prefill_tok_s']:.1f} decode {cpu['decode_tok_s']:.1f}", flush=True)
    assert gpu["tier"] == cpu["tier"]
    assert gpu["nonfinite_logits"] == 0 and cpu["nonfinite_logits"] == 0
    assert gpu["tokens"] == cpu["tokens"]
    assert gpu["last_logits"] == cpu["last_logits"]
    assert cpu["distinct_tokens"] >= gen // 4
