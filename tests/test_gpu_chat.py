"""The chat REPL's turn logic (chat_repl, chat.c:129-274) on the device
against the reference.

The reference side restates chat.c's loop in Python over the compiled
reference's own forward() and sample_greedy on the CPU: BOS only on a
conversation's first turn (:157-163), the user tokens through forward() at
current_pos, the reply token by token until max_tokens or EOS, current_pos
advanced by the prompt and the reply (the last sampled token counted, not
fed), and a restart at position 0 with BOS when a turn would not fit
(:169-190).  The device side drives gq_hip_chat_turn with the same inputs
and restarts on its -6.  Three turns (the third restarts the conversation)
on four layers of the TinyLlama-shape Q8_0 model and of the zero-mean
Q4_K_M one, whose greedy tokens vary from step to step; an EOS token taken
from the third turn's reply (and found nowhere before it) stops that turn
early.  The prompts run in prefill mode 1, token by token through the fp32
decode step (the reference's precision), where token parity is claimed;
prefill mode 0 (the bf16 prompt GEMM) is run too, for the positions and
the reply lengths, its token agreement printed.  Every reference forward() stays inside
the cache: chat.c's reply loop does not stop at max_seq, and the reference
engine asserts there (engine.c:422).  The reply tokens and the positions
after every turn must be identical."""
import ctypes as C
import dataclasses

import numpy as np
import pytest

from guanaco_amd import spec as S

pytestmark = pytest.mark.gpu

MAX_SEQ, MAX_TOKENS, BOS = 96, 24, 1


def cpu_chat(ref, rm, turns, eos):
    from oracle import fptr
    vocab = rm.mw.config.vocab_size
    pos, log = 0, []

    def fwd(toks, p):
        # the reference asserts past its cache (engine.c:422: chat.c's reply
        # does not stop at max_seq); the turns are chosen to stay inside
        assert p + len(toks) <= MAX_SEQ, (p, len(toks))
        arr = (C.c_int * len(toks))(*[int(t) for t in toks])
        out = ref.lib.forward(C.byref(rm.mw), rm.kv, rm.scratch, arr, len(toks), p, ref.vtable)
        lg = np.ctypeslib.as_array(C.cast(out.contents.data, C.POINTER(C.c_float)), shape=(vocab,)).copy()
        return int(ref.lib.sample_greedy(fptr(lg), vocab))

    for user in turns:
        toks = [BOS] + list(user) if pos == 0 else list(user)
        if pos + len(toks) >= MAX_SEQ - 1:
            pos = 0
            ref.lib.scratch_reset(rm.scratch)
            toks = [BOS] + list(user)
        nxt = fwd(toks, pos)
        pos += len(toks)
        reply, n = [nxt], 1
        for i in range(1, MAX_TOKENS):
            if n >= 512:
                break
            nxt = fwd([nxt], pos + i - 1)
            n += 1
            reply.append(nxt)
            if nxt == eos:
                break
        pos += n
        log.append((pos, reply))
    return log


def device_chat(dm, turns, eos):
    pos, log = 0, []
    for user in turns:
        toks = [BOS] + list(user) if pos == 0 else list(user)
        rc, reply, npos = dm.chat_turn(toks, pos, MAX_TOKENS, eos)
        if rc == -6:  # restart the conversation with BOS
            pos = 0
            rc, reply, npos = dm.chat_turn([BOS] + list(user), pos, MAX_TOKENS, eos)
        assert rc == 0, rc
        pos = npos
        log.append((pos, reply.tolist()))
    return log


@pytest.mark.parametrize("base", ["q8_0", "q4_k_m"])
def test_chat_three_turns_vs_reference(ref, orc, base):
    import guanaco_amd.hip as H
    from oracle import HostModel, RefModel
    spec = dataclasses.replace(S.TINYLLAMA_Q8 if base == "q8_0" else S.TINYLLAMA_ZM, name=f"chat-{base}-4-layers",
                               n_layers=4)
    rng = np.random.default_rng(5)
    turns = [rng.integers(3, spec.vocab, 20) for _ in range(3)]
    hm = HostModel(orc, spec, MAX_SEQ)
    kv0 = hm.new_kv()  # zeros, as the device cache starts
    rm = RefModel(ref, hm)
    rm.load_kv(kv0)
    plain = cpu_chat(ref, rm, turns, eos=-1)
    # turns 1-2 fill 21 + 24 + 20 + 24 = 89 positions: turn 3 restarts
    assert [p for p, _ in plain] == [45, 89, 45]
    seen = set(plain[0][1]) | set(plain[1][1])
    eos = next(t for i, t in enumerate(plain[2][1]) if i >= 4 and t not in seen and t not in plain[2][1][:i])
    rm.load_kv(kv0)
    cpu = cpu_chat(ref, rm, turns, eos)
    rm.close()
    assert cpu[:2] == plain[:2] and cpu[2][1][-1] == eos and len(cpu[2][1]) < MAX_TOKENS
    with H.Context(0) as ctx:
        dm = H.DeviceModel(ctx, spec, MAX_SEQ)
        assert H.lib.gq_hip_set_prefill_mode(ctx.h, 1) == 0
        dev = device_chat(dm, turns, eos)
        assert H.lib.gq_hip_set_prefill_mode(ctx.h, 0) == 1
        gemm = device_chat(dm, turns, -1)
    for t, (c, d) in enumerate(zip(cpu, dev)):
        print(f"turn {t}: reference pos {c[0]} reply {c[1]}; device pos {d[0]}")
        assert d[0] == c[0] and d[1] == c[1], t
    for t, (c, d) in enumerate(zip(plain, gemm)):
        same = sum(a == b for a, b in zip(c[1], d[1]))
        print(f"turn {t}, bf16 prompt GEMM: pos {d[0]}, {same} of {len(c[1])} reply tokens as the reference's")
        assert d[0] == c[0] and len(d[1]) == len(c[1]) and all(0 <= x < spec.vocab for x in d[1]), t


def test_chat_turn_rejects(ctx):
    import guanaco_amd.hip as H
    dm = H.DeviceModel(ctx, S.TINY_TEST, 32)
    assert dm.chat_turn([1] * 31, 0, 4, 2)[0] == -6      # does not fit: restart
    assert dm.chat_turn([1, 5, 6], 20, 16, -1)[0] == -5  # the reply runs past the cache
    assert dm.chat_turn([1, 5], 0, 4, 2, temperature=0.8)[0] == -1  # sampling needs rand() values
