"""The drop-in end to end on the GPU: the reference's own command-line
program, patched by guanaco_amd/host/reference-hip.patch and linked with the
HIP backend (oracle/build_ref_hip.sh), on GGUF files of the synthetic models
(tests/golden/gguf_writer.py).  With --device hip it runs the patched loader
(uploads), the bind in generate.c / chat.c, the per-layer engine hook and
the whole-model prompt and decode calls, and must print the tokens the same
program prints with --device cpu:
  * every layer on the device (whole-model decode), one layer (the
    --n-gpu-layers split: layer 0 through the engine hook, the rest and
    the sampler on the CPU, the LM head's vtable matvec on the device), and
    none;
  * greedy and sampled (top-k) decoding, and the chat REPL over two turns;
  * a model with an F32 LM head, which stays on the host while its layers
    run on the device.
Prompts run token by token in fp32 (GQ_HIP_PREFILL=steps) where tokens must
match the CPU's exactly; the default bf16 matrix-core prompt path is run on a
prompt whose first-token margin (1.68 on logits of standard deviation 3.5)
dwarfs its ~5e-3 relative error."""
import os

import pytest

import clitool
from guanaco_amd import spec as S

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not os.path.exists(clitool.CLI), reason="oracle/_ref/guanaco_hip not built")]

STEPS = {"GQ_HIP_PREFILL": "steps"}
N_TOK = 32


@pytest.fixture(scope="module")
def tinyllama_gguf(tmp_path_factory, orc):
    from gguf_writer import write_gguf
    path = str(tmp_path_factory.mktemp("gguf") / "tinyllama_zm.gguf")
    write_gguf(path, S.TINYLLAMA_ZM, 640, orc)
    return path


@pytest.fixture(scope="module")
def cpu_text(tinyllama_gguf):
    out, _ = clitool.run(tinyllama_gguf, prompt="Hello", max_tokens=N_TOK, device="cpu", threads=16)
    return clitool.generated_text(out)


@pytest.mark.parametrize("ngl,placement", [(None, "22 of 22 layers on the device, LM head on the device; prompts"),
                                           (1, "1 of 22 layers on the device, LM head on the device; forward()"),
                                           (0, "0 of 22 layers on the device, LM head on the host; forward()")])
def test_cli_hip_greedy_matches_cpu(tinyllama_gguf, cpu_text, ngl, placement):
    out, err = clitool.run(tinyllama_gguf, prompt="Hello", max_tokens=N_TOK, device="hip", n_gpu_layers=ngl,
                           threads=16, env=STEPS)
    assert "Backend: hip" in out
    assert placement in err, err
    got = clitool.generated_text(out)
    assert got == cpu_text
    assert len(set(clitool.text_to_ids(got))) > N_TOK // 2
    print(f"n_gpu_layers {ngl}: {clitool.decode_speed(out)} tok/s, tokens identical to --device cpu")


def test_cli_hip_topk_sampling_matches_cpu(tinyllama_gguf):
    """--temperature 0.7 --top-k 40 (the reference's defaults): the device
    sampler draws the same rand() values and picks the same tokens."""
    kw = dict(prompt="Hello", max_tokens=N_TOK, threads=16, temperature=0.7, extra=("--top-k", "40"))
    cpu, _ = clitool.run(tinyllama_gguf, device="cpu", **kw)
    hip, _ = clitool.run(tinyllama_gguf, device="hip", env=STEPS, **kw)
    assert clitool.generated_text(hip) == clitool.generated_text(cpu)


def test_cli_hip_matrix_core_prompt(tinyllama_gguf):
    """The default prompt path (bf16 GEMM chunks): same first token as the
    CPU on a prompt with a wide top-2 margin, and a full decode after it."""
    cpu, _ = clitool.run(tinyllama_gguf, prompt="Once upon a time", max_tokens=N_TOK, device="cpu", threads=16)
    hip, _ = clitool.run(tinyllama_gguf, prompt="Once upon a time", max_tokens=N_TOK, device="hip", threads=16)
    c, h = clitool.text_to_ids(clitool.generated_text(cpu)), clitool.text_to_ids(clitool.generated_text(hip))
    assert h[0] == c[0] and len(h) == len(c) == N_TOK
    same = next((i for i in range(N_TOK) if h[i] != c[i]), N_TOK)
    print(f"bf16 prompt path: first {same} of {N_TOK} tokens equal the CPU's")


def test_cli_hip_chat_matches_cpu(tinyllama_gguf):
    """chat_repl over two turns (KV reused, BOS only on the first): the HIP
    build prints the CPU build's replies."""
    stdin = "Hello\nTell me more\nexit\n"
    cpu, _ = clitool.run(tinyllama_gguf, prompt=None, max_tokens=16, device="cpu", threads=16,
                         extra=("--chat",), stdin=stdin)
    hip, err = clitool.run(tinyllama_gguf, prompt=None, max_tokens=16, device="hip", threads=16, env=STEPS,
                           extra=("--chat",), stdin=stdin)
    assert "prompts and decode steps run whole on the device" in err
    tail = lambda s: s[s.index("=== Chat Mode ==="):]
    assert tail(hip) == tail(cpu)
    assert tail(cpu).count("Assistant:") == 2


def test_cli_hip_f32_lm_head(tmp_path, orc):
    """An F32 LM head (loader.c:585 accepts it) stays on the host; the
    layers still run on the device through the engine hook."""
    from gguf_writer import write_gguf
    path = str(tmp_path / "f32_head.gguf")
    write_gguf(path, S.TINY_ZM, 64, orc, lm_head_f32=True)
    cpu, _ = clitool.run(path, prompt="Hello", max_tokens=24, device="cpu", threads=8)
    hip, err = clitool.run(path, prompt="Hello", max_tokens=24, device="hip", threads=8, env=STEPS)
    assert "2 of 2 layers on the device, LM head on the host" in err, err
    assert clitool.generated_text(hip) == clitool.generated_text(cpu)
