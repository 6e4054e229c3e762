"""The GGUF writer and the reference's own command-line program on CPU: a
synthetic model written by tests/golden/gguf_writer.py, loaded by the
reference's loader (loader.c:267-729) and decoded by its generate loop
(generate.c:96-330) with --device cpu, gives the oracle's greedy tokens for
the same model and prompt.  This pins the file writer the GPU command-line
tests (test_gpu_cli.py) build their models with."""
import os

import numpy as np
import pytest

import clitool
from guanaco_amd import spec as S

pytestmark = pytest.mark.skipif(not os.path.exists(clitool.CLI), reason="oracle/_ref/guanaco_hip not built")


def oracle_greedy(orc, spec, max_seq, prompt, n):
    from oracle import HostModel
    hm = HostModel(orc, spec, max_seq)
    kv = hm.new_kv()
    ids = clitool.prompt_ids(prompt)
    for pos, t in enumerate(ids):
        tok, _, _ = hm.forward(kv, t, pos)
    out = [tok]
    for i in range(1, n):
        tok, _, _ = hm.forward(kv, tok, len(ids) + i - 1)
        out.append(tok)
        if tok == 2:  # EOS ends generate()'s loop
            break
    return out


@pytest.mark.parametrize("prompt", ["Hello", "The quick brown fox"])
def test_gguf_cli_cpu_matches_oracle(tmp_path, orc, prompt):
    from gguf_writer import write_gguf
    spec, ms = S.TINY_ZM, 64
    path = str(tmp_path / "m.gguf")
    write_gguf(path, spec, ms, orc)
    out, _ = clitool.run(path, prompt=prompt, max_tokens=24, device="cpu", threads=4)
    got = clitool.text_to_ids(clitool.generated_text(out))
    want = oracle_greedy(orc, spec, ms, prompt, 24)
    assert got == want
    assert len(set(want)) > 4  # the zero-mean model's tokens vary


def test_gguf_header_and_offsets(tmp_path, orc):
    """The file as loader.c parses it: magic, version 3, the geometry keys,
    tensor data aligned to general.alignment."""
    import struct
    from gguf_writer import write_gguf
    path = str(tmp_path / "m.gguf")
    n = write_gguf(path, S.TINY_TEST, 64, orc)
    b = open(path, "rb").read()
    assert len(b) == n
    magic, ver, nt, nkv = struct.unpack("<IIQQ", b[:24])
    assert magic == 0x46554747 and ver == 3 and nt == 2 + 9 * S.TINY_TEST.n_layers + 1 and nkv == 12
    out, _ = clitool.run(path, max_tokens=2, device="cpu", threads=2)
    assert "H=512, heads=8, kv_heads=2, head_dim=64, layers=2, ff=1024, ctx=64, bos=1, eos=2" in out
    assert "All layer weights validated" in out
