"""GGUF v3 files of the synthetic models, for running the reference's own
command-line program (and its HIP build) end to end.

The format is what the reference's loader reads (loader.c:267-446): header
(magic "GGUF", version 3, tensor count, metadata count), metadata key/value
pairs (the llama.* geometry keys, general.alignment and the tokenizer keys
of loader.c:326-412), tensor infos (name, dims with the fastest-varying
first, ggml type, offset), padding to the alignment, then the tensor data.
Weights are the synthetic generator's bytes (guanaco_amd/csrc/gq_synth.h,
through the oracle), so a file holds exactly the model that
guanaco_amd.spec describes and that the oracle and the device build.

The vocabulary is made up: "<unk>", "<s>" (BOS 1), "</s>" (EOS 2), the 95
printable ASCII characters, then "[i]" for every other id, so any ASCII
prompt tokenizes and every generated token prints as distinct text.

Test infrastructure: tests and the profiling script call write_gguf; the
product never imports it.

    python tests/golden/gguf_writer.py <preset name> <max_seq> <path> [--lm-head-f32]
"""
import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (ROOT, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

from guanaco_amd import spec as S  # noqa: E402

GGUF_MAGIC = 0x46554747
ALIGN = 32
# GGUF metadata value types and ggml tensor types (loader.c:36-82)
T_UINT32, T_FLOAT32, T_STRING, T_ARRAY = 4, 6, 8, 9
GGML = {S.F32: 0, S.Q8_0: 8, S.Q4_K: 12, S.Q6_K: 14}
BOS, EOS = 1, 2


def vocab_strings(n):
    v = ["<unk>", "<s>", "</s>"] + [chr(c) for c in range(32, 127)]
    return (v + [f"[{i}]" for i in range(len(v), n)])[:n]


def _str(b, s):
    e = s.encode()
    b += struct.pack("<Q", len(e)) + e


def _kv_u32(b, k, v):
    _str(b, k)
    b += struct.pack("<II", T_UINT32, v)


def _tensor_list(spec, lm_head_f32):
    """(name, ggml dtype, dims fastest first, generator) in file order."""
    out = [("token_embd.weight", spec.embed_dtype, (spec.hidden, spec.vocab), ("q", -1, "embed"))]
    for l in range(spec.n_layers):
        dts = spec.dtypes(l)
        out.append((f"blk.{l}.attn_norm.weight", S.F32, (spec.hidden,), ("n", l, "rms_att")))
        for slot, name in (("wq", "attn_q"), ("wk", "attn_k"), ("wv", "attn_v"), ("wo", "attn_output")):
            rows, cols = spec.shape(slot)
            out.append((f"blk.{l}.{name}.weight", dts[slot], (cols, rows), ("q", l, slot)))
        out.append((f"blk.{l}.ffn_norm.weight", S.F32, (spec.hidden,), ("n", l, "rms_ffn")))
        for slot, name in (("wg", "ffn_gate"), ("wu", "ffn_up"), ("wd", "ffn_down")):
            rows, cols = spec.shape(slot)
            out.append((f"blk.{l}.{name}.weight", dts[slot], (cols, rows), ("q", l, slot)))
    out.append(("output_norm.weight", S.F32, (spec.hidden,), ("n", -1, "rms_final")))
    out.append(("output.weight", S.F32 if lm_head_f32 else spec.lm_head_dtype, (spec.hidden, spec.vocab),
                ("f" if lm_head_f32 else "q", -1, "lm_head")))
    return out


def _nbytes(dtype, dims):
    if dtype == S.F32:
        return 4 * int(np.prod(dims))
    return S.qbytes(dtype, dims[1], dims[0])


def lm_head_f32_values(orc, spec):
    """The F32 LM head of write_gguf(lm_head_f32=True): N(0,1) * 2^-4 (exact)."""
    seed = orc.tensor_seed(spec.seed, -1, S.SLOT["lm_head"])
    return np.ldexp(orc.synth_normal(seed, spec.vocab * spec.hidden), -4).astype(np.float32)


def write_gguf(path, spec, max_seq, orc, lm_head_f32=False):
    """Write `spec` as a GGUF v3 file at `path`; returns its size in bytes."""
    tensors = _tensor_list(spec, lm_head_f32)
    meta = bytearray()
    n_kv = 0
    _str(meta, "general.architecture")
    meta += struct.pack("<I", T_STRING)
    _str(meta, "llama")
    n_kv += 1
    for k, v in (("llama.embedding_length", spec.hidden), ("llama.attention.head_count", spec.n_heads),
                 ("llama.attention.head_count_kv", spec.n_kv_heads), ("llama.block_count", spec.n_layers),
                 ("llama.feed_forward_length", spec.ff), ("llama.context_length", max_seq),
                 ("general.alignment", ALIGN), ("tokenizer.ggml.bos_token_id", BOS),
                 ("tokenizer.ggml.eos_token_id", EOS)):
        _kv_u32(meta, k, v)
        n_kv += 1
    _str(meta, "tokenizer.ggml.tokens")
    voc = vocab_strings(spec.vocab)
    meta += struct.pack("<IIQ", T_ARRAY, T_STRING, len(voc))
    for t in voc:
        _str(meta, t)
    _str(meta, "tokenizer.ggml.scores")
    meta += struct.pack("<IIQ", T_ARRAY, T_FLOAT32, len(voc)) + np.zeros(len(voc), np.float32).tobytes()
    n_kv += 2
    infos = bytearray()
    off = 0
    offsets = []
    for name, dt, dims, _ in tensors:
        _str(infos, name)
        infos += struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
        infos += struct.pack("<IQ", GGML[dt], off)
        offsets.append(off)
        off += (_nbytes(dt, dims) + ALIGN - 1) // ALIGN * ALIGN
    head = struct.pack("<IIQQ", GGUF_MAGIC, 3, len(tensors), n_kv) + bytes(meta) + bytes(infos)
    data_start = (len(head) + ALIGN - 1) // ALIGN * ALIGN
    with open(path, "wb") as f:
        f.write(head + b"\0" * (data_start - len(head)))
        for (name, dt, dims, (kind, layer, slot)), o in zip(tensors, offsets):
            assert f.tell() == data_start + o, name
            seed = orc.tensor_seed(spec.seed, layer, S.SLOT[slot])
            if kind == "q":
                rows, cols = dims[1], dims[0]
                a = orc.synth_quant(spec.gen(dt), seed, rows, cols)
            elif kind == "n":
                a = orc.synth_norm_weight(seed, dims[0], spec.norm_shift)
            else:
                a = lm_head_f32_values(orc, spec)
            b = a.tobytes()
            f.write(b + b"\0" * ((-len(b)) % ALIGN))
        return f.tell()


if __name__ == "__main__":
    from oracle import Oracle
    name, max_seq, path = sys.argv[1], int(sys.argv[2]), sys.argv[3]
    n = write_gguf(path, S.PRESETS[name], max_seq, Oracle(), lm_head_f32="--lm-head-f32" in sys.argv)
    print(f"{path}: {n} bytes")
