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
    """Both GPU decode paths against the CPU reference: "seam" (the
    reference's slm_forward_step, every matmul a round trip) and "chain"
    (qk_decode.c: residual stream, norms, FFN and the greedy pick on the
    device). In the chain run every in-projection the reference's mixer
    asks for must be answered from the device results (its own host
    RMSNorm of h equals the device's bit for bit), and the host waits on
    the GPU only twice per layer plus once per token."""
    cpu = run(E2E_CPU, 240, prompt=prompt, gen=gen, seed=0)
    assert cpu["nonfinite_logits"] == 0
    assert cpu["distinct_tokens"] >= gen // 4
    for mode in ("seam", "chain"):
        # the pure drop-in (the reference's slm_forward_batch, one GPU call
        # per DeltaNet head and chunk) with the seam decode; qk_prefill.c's
        # one call per DeltaNet layer with the device decode step
        prefill = "seam" if mode == "seam" else "layer"
        gpu = run(E2E_GPU, 240, prompt=prompt, gen=gen, seed=0, decode=mode, prefill=prefill)
        print(f"[e2e] gpu-{mode} prefill ({prefill}) {gpu['prefill_tok_s']:.1f} tok/s, "
              f"{gpu['prefill_gpu_matmul_s']:.3f} s in matmul calls, {gpu['prefill_gpu_deltanet_s']:.3f} s in "
              f"DeltaNet calls; decode {gpu['decode_tok_s']:.1f} tok/s "
              f"({gpu['host_syncs_per_token']:.1f} host syncs/token); cpu prefill {cpu['prefill_tok_s']:.1f} "
              f"decode {cpu['decode_tok_s']:.1f}", flush=True)
        assert gpu["tier"] == cpu["tier"]
        assert gpu["nonfinite_logits"] == 0
        assert gpu["prefill_path"] == f"gpu-{prefill}"
        assert gpu["prefill_logits"] == cpu["prefill_logits"], mode
        assert gpu["tokens"] == cpu["tokens"], mode
        assert gpu["last_logits"] == cpu["last_logits"], mode
        if mode == "chain":
            layers = gpu["layers"]
            assert gpu["prefetch_misses"] == 0
            assert gpu["prefetch_hits"] == gen * (layers * 4 - layers // 4)    # 4 per SSM layer, 3 per attention
            assert gpu["host_syncs_per_token"] == 2 * layers + 1


@pytest.mark.gpu
def test_e2e_sampled_tokens_identical():
    """The reference's default sampler chain (T 0.7, top-k 40, top-p 0.9,
    min-p 0.05, repetition penalty 1.25 over 64) with a fixed rng seed:
    the chain run samples on the device (hip_sample), the seam run and the
    CPU reference with sample_with on the host; the token streams must be
    identical."""
    cpu = run(E2E_CPU, 240, prompt=64, gen=48, seed=0, sample=11)
    assert cpu["sampler"] == "slm_sampler_defaults" and cpu["distinct_tokens"] >= 12
    for mode in ("seam", "chain"):
        gpu = run(E2E_GPU, 240, prompt=64, gen=48, seed=0, sample=11, decode=mode)
        print(f"[e2e] sampled gpu-{mode} decode {gpu['decode_tok_s']:.1f} tok/s; cpu {cpu['decode_tok_s']:.1f}",
              flush=True)
        assert gpu["tokens"] == cpu["tokens"], mode
        assert gpu["last_logits"] == cpu["last_logits"], mode


# ---- GGUF round trip ------------------------------------------------------------
# qwen_e2e --write-gguf writes the random model as GGUF v3 (host/gguf_write.c);
# --gguf loads a file through the reference's own slm_model_load. The token
# stream from the loaded file must equal the built model's, and the file
# must parse under an independent reader of the GGUF v3 layout.

def read_gguf(path):
    """Minimal GGUF v3 reader for the test: header, key/values, tensor infos."""
    import struct
    with open(path, "rb") as f:
        buf = f.read(1 << 24)                       # header sections only
        size = os.fstat(f.fileno()).st_size
    pos = 0

    def take(fmt):
        nonlocal pos
        v = struct.unpack_from("<" + fmt, buf, pos)
        pos += struct.calcsize("<" + fmt)
        return v[0] if len(v) == 1 else v

    def string():
        nonlocal pos
        n = take("Q")
        s = buf[pos:pos + n].decode()
        pos += n
        return s

    def value(t):
        if t == 4:
            return take("I")
        if t == 5:
            return take("i")
        if t == 6:
            return take("f")
        if t == 8:
            return string()
        if t == 9:
            et, n = take("I"), take("Q")
            return [value(et) for _ in range(n)]
        raise AssertionError(f"unexpected value type {t}")

    assert take("I") == 0x46554747 and take("I") == 3
    n_t, n_kv = take("Q"), take("Q")
    kv = {}
    for _ in range(n_kv):
        k = string()
        kv[k] = value(take("I"))
    tensors = {}
    for _ in range(n_t):
        name = string()
        nd = take("I")
        shape = [take("Q") for _ in range(nd)]
        tensors[name] = (shape, take("I"), take("Q"))
    align = kv.get("general.alignment", 32)
    data_start = (pos + align - 1) // align * align
    return kv, tensors, data_start, size


BLOCK = {0: (1, 4), 8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210)}


def test_gguf_roundtrip_cpu(tmp_path):
    path = str(tmp_path / "e2e.gguf")
    built = run(E2E_CPU, 120, prompt=12, gen=6, layers=4, seed=5, **{"write-gguf": path})
    kv, tensors, data_start, size = read_gguf(path)
    assert kv["general.architecture"] == "qwen35"
    assert kv["qwen35.block_count"] == 4 and kv["qwen35.embedding_length"] == 1024
    assert kv["qwen35.rope.dimension_sections"] == [11, 11, 10, 0]
    assert len(kv["tokenizer.ggml.tokens"]) == 248320
    # token_embd and output_norm, 14 tensors per DeltaNet layer (layers
    # 0-2) and 11 per attention layer (layer 3)
    assert len(tensors) == 2 + 3 * 14 + 11
    end = 0
    for name, (shape, ttype, off) in tensors.items():
        elems, bb = BLOCK[ttype]
        n = 1
        for d in shape:
            n *= d
        assert n % elems == 0, name
        assert off % kv["general.alignment"] == 0, name
        end = max(end, data_start + off + n // elems * bb)
    assert tensors["token_embd.weight"][:2] == ([1024, 248320], 14)
    assert tensors["blk.0.ssm_alpha.weight"][:2] == ([1024, 16], 8)
    assert end == size
    loaded = run(E2E_CPU, 120, prompt=12, gen=6, layers=4, seed=5, gguf=path)
    assert loaded["source"] == "gguf" and built["source"] == "built"
    assert loaded["tokens"] == built["tokens"]
    assert loaded["last_logits"] == built["last_logits"]


@pytest.mark.gpu
def test_gguf_gpu_tokens_identical(tmp_path):
    path = str(tmp_path / "e2e.gguf")
    cpu = run(E2E_CPU, 120, prompt=24, gen=8, layers=4, seed=6, **{"write-gguf": path})
    gpu = run(E2E_GPU, 120, prompt=24, gen=8, layers=4, seed=6, gguf=path)
    assert gpu["source"] == "gguf"
    assert gpu["tokens"] == cpu["tokens"]
    assert gpu["last_logits"] == cpu["last_logits"]


# ---- the reference's own generation loop through the one-line binding -----------
# slm_drive.c includes the reference's TU root slm/slm.c (with qk_seam.c in
# front for the GPU build, host/_build/slm_drive_gpu; unchanged for the CPU
# twin, oracle/_ref/slm_drive_cpu) and calls slm_generate_raw
# (slm/slm.c:237-358) on token ids over a GGUF file written by qwen_e2e.
# The generated ids come from the reference's own token trace.
DRIVE_CPU = os.path.join(ROOT, "oracle", "_ref", "slm_drive_cpu")
DRIVE_GPU = os.path.join(ROOT, "qwen.haiku_amd", "host", "_build", "slm_drive_gpu")


def drive(path, gguf, timeout=300, flags=(), **kw):
    if not os.path.exists(path):
        pytest.fail(f"{path} is not built (make -C oracle; make -C qwen.haiku_amd/host)")
    args = [path, "--gguf", gguf] + list(flags)
    for k, v in kw.items():
        args += [f"--{k.replace('_', '-')}", str(v)]
    print(f"[e2e] {' '.join(os.path.relpath(a, ROOT) if a == path else a for a in args)}", flush=True)
    r = subprocess.run(args, capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0, f"{path} failed ({r.returncode}):\n{r.stderr[-2000:]}"
    toks = [int(ln.split()[1]) for ln in r.stderr.splitlines() if ln.startswith("[tok] ")]
    return json.loads(r.stdout.strip().splitlines()[-1]), toks


@pytest.fixture(scope="module")
def drive_gguf(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("drive") / "m4.gguf")
    run(E2E_CPU, 120, prompt=48, gen=48, layers=4, seed=8, **{"write-gguf": path})   # max_position 97
    return path


def test_slm_drive_cpu_deterministic(drive_gguf):
    a, ta = drive(DRIVE_CPU, drive_gguf, prompt=24, gen=12, seed=2)
    b, tb = drive(DRIVE_CPU, drive_gguf, prompt=24, gen=12, seed=2)
    assert ta == tb and a["generated"] == len(ta) == 12
    assert len(set(ta)) > 1


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["greedy", "batch", "sampled"])
def test_slm_generate_raw_through_seam(drive_gguf, mode):
    """The reference's slm_generate_raw, prefill (per token, or
    slm_forward_batch) and decode loop unchanged, with the seam in front:
    the token stream must equal the unchanged reference's."""
    flags = ("--batch",) if mode != "greedy" else ()
    kw = dict(prompt=32, gen=40, seed=5)
    if mode == "sampled":
        kw.update(sample=11, min_new=6)
    cpu, tc = drive(DRIVE_CPU, drive_gguf, flags=flags, **kw)
    gpu, tg = drive(DRIVE_GPU, drive_gguf, flags=flags, **kw)
    assert tc and tg == tc
    assert gpu["generated"] == cpu["generated"] == len(tc)
