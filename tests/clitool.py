"""Running the reference's command-line program (oracle/_ref/guanaco_hip: the
reference with guanaco_amd/host/reference-hip.patch and the HIP backend, built
by oracle/build_ref_hip.sh) on GGUF files from tests/golden/gguf_writer.py,
and reading its output back as token ids."""
import os
import re
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "oracle", "_ref", "guanaco_hip")


def run(model, prompt="Hello", max_tokens=16, device="cpu", n_gpu_layers=None, threads=8, env=None,
        extra=(), stdin=None, timeout=600, temperature=0.0):
    """Runs the program; returns (stdout, stderr).  Raises on a non-zero exit."""
    cmd = [CLI, "--model", model, "--max-tokens", str(max_tokens), "--temperature", str(temperature),
           "--device", device, "--threads", str(threads)]
    if prompt is not None:
        cmd += ["--prompt", prompt]
    if n_gpu_layers is not None:
        cmd += ["--n-gpu-layers", str(n_gpu_layers)]
    cmd += list(extra)
    e = dict(os.environ)
    e.update(env or {})
    p = subprocess.run(cmd, capture_output=True, text=True, env=e, input=stdin, timeout=timeout)
    if p.returncode != 0:
        raise RuntimeError(f"{' '.join(cmd)} exited {p.returncode}:\n{p.stdout[-2000:]}\n{p.stderr[-2000:]}")
    return p.stdout, p.stderr


def generated_text(out):
    """The tokens generate() printed: between its "Generating N tokens..."
    line and the stats (generate.c:170-171, :326-330)."""
    m = re.search(r"Generating \d+ tokens\.\.\.\n\n(.*)\n\n--- Stats ---", out, re.S)
    if not m:
        raise ValueError("no generated text in:\n" + out[-2000:])
    return m.group(1)


def decode_speed(out):
    m = re.search(r"Decode speed: ([0-9.]+) tok/s", out)
    return float(m.group(1)) if m else None


def text_to_ids(text):
    """Token ids of text printed with gguf_writer's vocabulary: "<unk>",
    "<s>", "</s>", the printable ASCII characters (ids 3..97), "[i]" for
    i >= 98."""
    ids, i = [], 0
    while i < len(text):
        m = re.match(r"\[(\d+)\]", text[i:])
        if m and int(m.group(1)) >= 98:
            ids.append(int(m.group(1)))
            i += m.end()
            continue
        if text[i] == "\n":  # generate() prints EOS as a newline (generate.c:318-321)
            ids.append(2)
            i += 1
            continue
        for s, t in (("<unk>", 0), ("</s>", 2), ("<s>", 1)):
            if text.startswith(s, i):
                ids.append(t)
                i += len(s)
                break
        else:
            ids.append(ord(text[i]) - 32 + 3)
            i += 1
    return ids


def prompt_ids(prompt):
    """tokenize() of an ASCII prompt with gguf_writer's vocabulary: BOS, then
    one token per character (tokenizer.c's longest-prefix match finds no
    longer piece)."""
    return [1] + [ord(c) - 32 + 3 for c in prompt]
