"""The reference-shaped C++ API (include/infengine/*.h) compiles with the host
compiler, links against libinfengine_amd.so and (GPU) produces the same tokens
as the Python-driven entry points."""
import os
import pathlib
import subprocess

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
LIBDIR = ROOT / "infengine_amd"


def build_manager(out_dir: pathlib.Path, name: str = "manager_main") -> pathlib.Path:
    exe = out_dir / name
    cmd = ["g++", "-std=c++17", "-O2", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__",
           f"-I{ROOT / 'include'}", "-I/opt/rocm/include", str(ROOT / f"tests/cpp/{name}.cpp"),
           f"-L{LIBDIR}", "-linfengine_amd", "-L/opt/rocm/lib", "-lamdhip64",
           f"-Wl,-rpath,{LIBDIR}", "-Wl,-rpath,/opt/rocm/lib", "-o", str(exe)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    return exe


@pytest.mark.parametrize("name", ["manager_main", "batcher_main", "sampling_main"])
def test_cpp_api_compiles_and_links(tmp_path, hip, name):
    exe = build_manager(tmp_path, name)
    assert exe.exists()


@pytest.mark.gpu
def test_cpp_continuous_batcher(tmp_path, hip):
    """The continuous batcher over the paged KV cache: four requests admitted at once, joining at
    different steps, and one at a time produce the same tokens (the program checks and prints
    OK), and every page returns to the pool; with EOS ids each request stops right after its
    EOS; a prefill that fails leaves its request queued and loses no page."""
    from gpu_util import say
    exe = build_manager(tmp_path, "batcher_main")
    say("C++ ContinuousBatcher: 4 requests, 3 schedules")
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    lines = res.stdout.splitlines()
    assert lines[-1] == "OK", res.stdout
    assert [len(l.split()) - 2 for l in lines if l.startswith("tokens")] == [12, 10, 14, 16]
    assert sum(l.startswith("eos") for l in lines) == 4


@pytest.mark.gpu
def test_cpp_manager_matches_python_driver(tmp_path, hip):
    import torch
    from gpu_util import say
    from infengine_amd.engine import Context, ModelWeights, Request
    exe = build_manager(tmp_path)
    say("C++ Manager: prompt 16, 8 new tokens")
    res = subprocess.run([str(exe), "16", "8", "7"], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr
    cpp_tokens = [int(t) for t in res.stdout.splitlines()[0].split()[1:]]
    assert len(cpp_tokens) == 8
    # the same request through the Python-driven C-ABI
    c = Context(0)
    W = ModelWeights.random_init(seed=7, std=0.02)
    req = Request(c, W, max_seq_len=64)
    prompt = [(i * 7919 + 17) % 128256 for i in range(16)]
    req.tokens[:16] = torch.tensor(prompt, dtype=torch.int32, device="cuda")
    toks = [req.prefill(16)]
    for n in range(1, 8):
        req.tokens[16 + n - 1] = toks[-1]
        toks.append(req.decode_step(16 + n))
    W.free()
    c.close()
    assert cpp_tokens == toks
    # the same request with an EOS id: stops right after its first occurrence
    eos = toks[4]
    stop = toks.index(eos) + 1
    res = subprocess.run([str(exe), "16", "8", "7", str(eos)], capture_output=True, text=True,
                         timeout=300)
    assert res.returncode == 0, res.stderr
    assert [int(t) for t in res.stdout.splitlines()[0].split()[1:]] == toks[:stop]


@pytest.mark.gpu
def test_cpp_handle_free_sample_token_amax(tmp_path, hip):
    """The reference's argmax test (tests/test_sampling.cu) in C++: runtime-allocated buffers and
    the handle-free sample_token_amax(d_logits, d_output) (sampling.cuh:4) on the torch.argmax
    fixture rows (ties, NaN, signed zeros), each id bit-exact."""
    from gpu_util import say
    exe = build_manager(tmp_path, "sampling_main")
    g = np.load(ROOT / "tests/golden/argmax_torch.npz")
    for i, (row, want) in enumerate(zip(g["logits"], g["expect"])):
        f = tmp_path / f"logits{i}.f32"
        np.ascontiguousarray(row, dtype=np.float32).tofile(f)
        say(f"C++ sample_token_amax, fixture row {i}")
        res = subprocess.run([str(exe), str(f)], capture_output=True, text=True, timeout=120)
        assert res.returncode == 0, res.stderr
        assert int(res.stdout.split()[0]) == int(want), (i, res.stdout)
