"""Synthetic model geometries of the decode hot path.

A ``ModelSpec`` names the shape of a Llama-family model as the reference
loader describes it (``types.h:110-147``: ``ModelConfig`` / ``LayerWeights``),
the storage dtype of every weight, and the seed from which every weight byte,
norm weight and KV pre-fill value is derived (``csrc/gq_synth.h``).  The same
spec drives the device fill kernels (bench, GPU tests) and the CPU oracle, so
both sides see bit-identical inputs without shipping weights.

Weights use the reference's ``[rows = out_features][cols = in_features]``
convention (``loader.c:503-510``).
"""
from __future__ import annotations

from dataclasses import dataclass, field

# dtype codes of the reference's DataType enum (types.h:16-24)
F32, Q8_0, Q4_K, Q6_K = 0, 2, 4, 5
BLOCK = {Q4_K: (256, 144), Q6_K: (256, 210), Q8_0: (32, 34)}
DTYPE_NAME = {F32: "f32", Q8_0: "q8_0", Q4_K: "q4_k", Q6_K: "q6_k"}

# generator code of the zero-mean Q4_K rule (gq_synth.h gq_q4k_zm_byte): or'ed
# into the Q4_K dtype code
SYNTH_Q4K_ZERO_MEAN = 0x100

# tensor slots of gq_tensor_seed()
SLOT = dict(wq=0, wk=1, wv=2, wo=3, wg=4, wu=5, wd=6, rms_att=7, rms_ffn=8,
            embed=10, lm_head=11, rms_final=12, kv_k=13, kv_v=14, act=15)
LAYER_WEIGHTS = ("wq", "wk", "wv", "wo", "wg", "wu", "wd")


def qbytes(dtype: int, rows: int, cols: int) -> int:
    qk, bb = BLOCK[dtype]
    assert cols % qk == 0, (dtype, cols)
    return rows * (cols // qk) * bb


@dataclass
class ModelSpec:
    name: str
    n_layers: int
    hidden: int
    ff: int
    n_heads: int
    n_kv_heads: int
    vocab: int
    # per-layer dtype rule: dict slot -> dtype, or callable(layer) -> dict
    layer_dtypes: object = None
    embed_dtype: int = Q4_K
    lm_head_dtype: int = Q6_K
    # the reference hard-codes theta=500000 (kernels_cpu.c:408) and
    # eps=1e-6 (engine.c:359,524,582); parity runs use those values
    rope_theta: float = 500000.0
    rms_eps: float = 1e-6
    seed: int = 0x5EED
    # Q4_K tensors from the zero-mean rule (gq_q4k_zm_byte) instead of the
    # plain one; the blocks are Q4_K either way
    q4k_zero_mean: bool = False
    # RMSNorm weights (1 + N(0,1)/64) * 2^-norm_shift (exact): the activation
    # scale every matvec and the attention scores see
    norm_shift: int = 0
    head_dim: int = field(init=False)

    def __post_init__(self):
        assert self.hidden % self.n_heads == 0
        self.head_dim = self.hidden // self.n_heads  # loader.c:415-417

    def dtypes(self, layer: int) -> dict:
        rule = self.layer_dtypes
        d = rule(layer) if callable(rule) else dict(rule)
        return {k: d.get(k, Q4_K) for k in LAYER_WEIGHTS}

    def gen(self, dtype: int) -> int:
        """Generator code of a tensor of this dtype (gq_hip_synth_quant)."""
        return dtype | SYNTH_Q4K_ZERO_MEAN if (dtype == Q4_K and self.q4k_zero_mean) else dtype

    def shape(self, slot: str) -> tuple:
        H, F, kvd = self.hidden, self.ff, self.n_kv_heads * self.head_dim
        return dict(wq=(H, H), wk=(kvd, H), wv=(kvd, H), wo=(H, H), wg=(F, H),
                    wu=(F, H), wd=(H, F), embed=(self.vocab, H),
                    lm_head=(self.vocab, H))[slot]

    def weight_bytes_per_token(self) -> int:
        """Algorithmic weight bytes streamed per decode token."""
        tot = 0
        for l in range(self.n_layers):
            for k, dt in self.dtypes(l).items():
                tot += qbytes(dt, *self.shape(k))
        tot += qbytes(self.lm_head_dtype, *self.shape("lm_head"))
        tot += 4 * self.hidden * (2 * self.n_layers + 1)  # norm weights
        tot += qbytes(self.embed_dtype, 1, self.hidden)  # one embedding row
        return tot

    def kv_bytes_per_token(self, pos: int) -> int:
        """K+V bytes attention reads at position pos (pos+1 rows), all layers."""
        return 2 * self.n_layers * self.n_kv_heads * (pos + 1) * self.head_dim * 4


def _q6k_on_even(layer):
    # "Q6_K on half the attn_v/ffn_down layers": the even layers
    return dict(wv=Q6_K, wd=Q6_K) if layer % 2 == 0 else {}


LLAMA8B = ModelSpec("llama-3.1-8b-shape-q4_k_m", n_layers=32, hidden=4096, ff=14336,
                    n_heads=32, n_kv_heads=8, vocab=128256, layer_dtypes=_q6k_on_even)

TINYLLAMA = ModelSpec("tinyllama-1.1b-shape", n_layers=22, hidden=2048, ff=5632,
                      n_heads=32, n_kv_heads=4, vocab=32000,
                      layer_dtypes=dict(wv=Q6_K, wd=Q6_K))

# TinyLlama shape with every weight Q8_0 (embedding and LM head included):
# zero-mean weights.  The Q4_K generator's weights have a positive mean
# (d sc q - dmin m with q in 0..15), which gives every hidden state a large
# common component; the LM head then ranks tokens by a fixed per-row bias and
# the greedy chain repeats one or two tokens.  This variant's tokens vary at
# every step with top-2 margins of O(1)-O(10) on logits of standard
# deviation ~100, so token identity discriminates.
TINYLLAMA_Q8 = ModelSpec("tinyllama-1.1b-shape-q8_0", n_layers=22, hidden=2048, ff=5632,
                         n_heads=32, n_kv_heads=4, vocab=32000,
                         layer_dtypes={k: Q8_0 for k in LAYER_WEIGHTS}, embed_dtype=Q8_0,
                         lm_head_dtype=Q8_0)

# Zero-mean Q4_K_M variants of the two BASELINE shapes, for token parity that
# discriminates on the Q4_K / Q6_K kernels the benchmark runs: the same dtype
# mix as TINYLLAMA / LLAMA8B with every Q4_K tensor from the zero-mean rule,
# and norm weights scaled by 2^-7 so attention scores stay O(1)-O(10)
# (with the unscaled weights q and k entries reach ~300 and the softmax is a
# hard maximum whose ties hinge on fp32 rounding).
TINYLLAMA_ZM = ModelSpec("tinyllama-1.1b-shape-q4_k_m-zero-mean", n_layers=22, hidden=2048, ff=5632,
                         n_heads=32, n_kv_heads=4, vocab=32000,
                         layer_dtypes=dict(wv=Q6_K, wd=Q6_K), q4k_zero_mean=True, norm_shift=7)
LLAMA8B_ZM = ModelSpec("llama-3.1-8b-shape-q4_k_m-zero-mean", n_layers=32, hidden=4096, ff=14336,
                       n_heads=32, n_kv_heads=8, vocab=128256, layer_dtypes=_q6k_on_even,
                       q4k_zero_mean=True, norm_shift=7)

# small model used by the quick parity tests: same mixed-dtype rule as the 8B
# shape, GQA 4:1 like both presets, head_dim 64
TINY_TEST = ModelSpec("tiny-test", n_layers=2, hidden=512, ff=1024, n_heads=8,
                      n_kv_heads=2, vocab=1000, layer_dtypes=_q6k_on_even)

# the tiny model with zero-mean Q4_K weights and scaled norms (as the *_ZM
# presets): its greedy tokens vary, for the command-line tests
TINY_ZM = ModelSpec("tiny-test-zero-mean", n_layers=2, hidden=512, ff=1024, n_heads=8,
                    n_kv_heads=2, vocab=1000, layer_dtypes=_q6k_on_even, q4k_zero_mean=True, norm_shift=7)

# the tiny model with a 28672-wide FFN (Llama-2-70B's ff): the down
# projection's rows are longer than 16384 columns
WIDE_FF_TEST = ModelSpec("wide-ff-test", n_layers=2, hidden=512, ff=28672, n_heads=8,
                         n_kv_heads=2, vocab=1000, layer_dtypes=_q6k_on_even)

PRESETS = {s.name: s for s in (LLAMA8B, TINYLLAMA, TINYLLAMA_Q8, TINYLLAMA_ZM, LLAMA8B_ZM, TINY_TEST,
                               TINY_ZM, WIDE_FF_TEST)}
