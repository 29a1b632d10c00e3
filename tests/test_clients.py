"""The drop-in boundary as a caller of the reference sees it: two client programs compiled against include/ and
linked with libctorch_amd.so, with no Python in between.

  tests/clients/decode_client.c    C17: the decoder block of the reference's tests/c_api.c:28-42 (on DL_CUDA),
                                   then the greedy loop of examples/decoder_generate.cpp:16-31 over the C surface;
  tests/clients/decode_client.cpp  C++20: greedy byte generation through the dl:: C++ API a reference caller
                                   uses (Device::cuda(), NoGradGuard, io::load, load_state_dict, make_cache,
                                   decode, from_span, select, argmax().item(), full).

The CPU test compiles both with -Werror; the GPU test runs the programs __graft_entry__.build() built (under
tests/clients/_build) on a byte decoder whose weights the oracle also evaluates, and requires the oracle's greedy
bytes (f32: identical ids)."""
import os
import shutil
import subprocess

import numpy as np
import pytest

import ctorch_amd as ct
import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLIENTS = os.path.join(ROOT, "tests", "clients")
BUILT = os.path.join(CLIENTS, "_build")
BYTE_DECODER = oracle.ModelConfig(vocab=256, layers=2, dimensions=64, heads=4, kv_heads=2, hidden=256, context=128,
                                  dtype="f32")


def test_clients_compile_against_the_public_headers(tmp_path):
    lib = os.path.join(ROOT, "ctorch_amd")
    link = ["-L" + lib, "-lctorch_amd", "-Wl,-rpath," + lib]
    for compiler, std, source, flags in (("gcc", "-std=c17", "decode_client.c", ["-Wpedantic"]),
                                         ("g++", "-std=c++20", "decode_client.cpp", [])):
        if shutil.which(compiler) is None:
            pytest.skip(f"{compiler} is not installed")
        out = tmp_path / source.replace(".", "_")
        cmd = [compiler, std, "-O1", "-Wall", "-Wextra", "-Werror", *flags, "-I" + os.path.join(ROOT, "include"),
               os.path.join(CLIENTS, source), "-o", str(out), *link]
        result = subprocess.run(cmd, capture_output=True, text=True)
        assert result.returncode == 0, result.stderr
        assert out.exists()


def byte_decoder_archive(path, root=(303, 0)):
    """The byte decoder's state (tokens.weight, decoder.*, output.weight tied to tokens.weight) as a .ct archive,
    and the oracle over the same weights."""
    weights = oracle.synthesize_weights(BYTE_DECODER, root, 0.05)
    weights["output.weight"] = weights["tokens.weight"]
    cfg = BYTE_DECODER
    host = ct.transformer_decoder(cfg.layers, cfg.dimensions, cfg.heads, cfg.kv_heads, cfg.hidden, cfg.context,
                                  ct.F32, ct.device("cpu"))
    state = {"tokens.weight": weights["tokens.weight"]}
    for name, tensor in host.state().items():  # registration order; the RoPE buffers come from the library
        state["decoder." + name] = weights.get("decoder." + name, tensor)
    state["output.weight"] = weights["output.weight"]
    ct.save_state(str(path), state)
    return oracle.OracleLM(cfg, weights)


def run_client(args):
    if not os.path.exists(args[0]):
        pytest.fail(f"{args[0]} is not built: run __graft_entry__.build() (make -C tests/clients)")
    result = subprocess.run(args, capture_output=True, text=True, timeout=120)
    assert result.returncode == 0, (args, result.stdout, result.stderr)
    return result.stdout


@pytest.mark.gpu
def test_c17_client_runs_the_reference_block_and_the_greedy_loop(tmp_path):
    print("case: C17 client (tests/c_api.c decoder block on DL_CUDA, greedy loop over the C surface)", flush=True)
    ref = byte_decoder_archive(tmp_path / "byte_decoder.ct")
    prefix = "the MI355X decodes "
    out = run_client([os.path.join(BUILT, "decode_client_c"), str(tmp_path / "byte_decoder.ct"), prefix, "24"])
    lines = out.split("\n")
    assert lines[0] == "reference block: cache length 2"
    got = np.array([int(x) for x in lines[1:] if x])
    want, _ = ref.generate(np.frombuffer(prefix.encode(), np.uint8).astype(np.int64).reshape(1, -1), 24)
    assert np.array_equal(got, want[0]), (got, want[0])


@pytest.mark.gpu
def test_cpp20_client_generates_through_the_cpp_api_on_device_cuda(tmp_path):
    print("case: C++20 client (dl:: decoder API with Device::cuda() and NoGradGuard)", flush=True)
    ref = byte_decoder_archive(tmp_path / "byte_decoder.ct", root=(304, 0))
    prefix = "tokens per second "
    out = run_client([os.path.join(BUILT, "decode_client_cpp"), "--archive", str(tmp_path / "byte_decoder.ct"),
                      "--prompt", prefix, "--steps", "24", "--device", "cuda"])
    lines = out.split()
    assert lines[-1] == f"cache_length={len(prefix) + 23}"
    got = np.array([int(x) for x in lines[:-1]])
    want, _ = ref.generate(np.frombuffer(prefix.encode(), np.uint8).astype(np.int64).reshape(1, -1), 24)
    assert np.array_equal(got, want[0]), (got, want[0])
