"""Inputs of the golden fixtures: seeds, shapes and generators shared by
tests/golden/make_golden.py (which records the reference's outputs) and the
tests (which regenerate the same inputs and compare)."""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "forword.c_amd"))
import fwgpu  # noqa: E402

Q4, Q5, Q8 = fwgpu.GGML_Q4_0, fwgpu.GGML_Q5_0, fwgpu.GGML_Q8_0
Q4K, Q6K = fwgpu.GGML_Q4_K, fwgpu.GGML_Q6_K

# Model fixtures.  "tiny": dim 288, ffn 768, 6 layers, 6/6 heads, vocab 32000,
# ctx 256, all Q8_0, theta 1e4, 16-token prompt + 128 greedy tokens.  "gqa":
# 8 query / 2 KV heads (group 4).  "q5": Q5_0 linears, embedding and output.
# "qwen2": architecture qwen2 (q/k/v biases, RoPE base raised to 1e6 by the
# config loader), 8/2 heads, Q8_0 linears.  "gemma": gated FFN with the tanh
# GELU, embedding rows times sqrt(n_embd), lm-head tied to token_embd.
# "phi2": LayerNorm with biases, parallel residual, plain GELU-tanh FFN,
# NEOX RoPE, attn_output bias; 4 heads of 64.  "gpt2": LayerNorm, fused
# attn_qkv with bias, learned position embeddings, no RoPE, plain erf-GELU FFN
# with biases, lm-head tied to token_embd.
MODELS = {
    "tiny": {"spec": lambda: fwgpu.spec_tiny(seed=20240601), "n_prompt": 16, "n_gen": 128,
             "max_ctx": 0, "prompt_seed": 1},
    "gqa": {"spec": lambda: fwgpu.spec(256, 512, 2, 8, 2, 1000, 64, 10000.0, seed=77),
            "n_prompt": 8, "n_gen": 24, "max_ctx": 0, "prompt_seed": 2},
    "q5": {"spec": lambda: fwgpu.spec(288, 768, 2, 6, 6, 4096, 64, 10000.0, linear_type=Q5,
                                      embd_type=Q5, output_type=Q5, seed=55),
           "n_prompt": 8, "n_gen": 24, "max_ctx": 0, "prompt_seed": 3},
    "qwen2": {"spec": lambda: fwgpu.spec(256, 512, 2, 8, 2, 1000, 64, 10000.0, seed=99,
                                         arch="qwen2"),
              "n_prompt": 8, "n_gen": 24, "max_ctx": 0, "prompt_seed": 4},
    "gemma": {"spec": lambda: fwgpu.spec(256, 512, 2, 8, 2, 1000, 64, 10000.0, seed=123, arch="gemma"),
              "n_prompt": 8, "n_gen": 24, "max_ctx": 0, "prompt_seed": 5},
    "phi2": {"spec": lambda: fwgpu.spec(256, 1024, 2, 4, 4, 1000, 64, 10000.0, seed=321, arch="phi2"),
             "n_prompt": 8, "n_gen": 24, "max_ctx": 0, "prompt_seed": 6},
    "gpt2": {"spec": lambda: fwgpu.spec(256, 1024, 2, 4, 4, 1000, 64, 10000.0, seed=654, arch="gpt2"),
             "n_prompt": 8, "n_gen": 24, "max_ctx": 0, "prompt_seed": 7},
}


def prompt(name) -> np.ndarray:
    m = MODELS[name]
    vocab = m["spec"]().n_vocab
    return np.random.default_rng(m["prompt_seed"]).integers(3, vocab, m["n_prompt"]).astype(np.uint32)


def n_forwards(name) -> int:
    return MODELS[name]["n_prompt"] + MODELS[name]["n_gen"] - 1


def logit_steps(name):
    n = n_forwards(name)
    return [0, MODELS[name]["n_prompt"] - 1, n - 1]


def trace_steps(name):
    return [0, n_forwards(name) - 1]


# quant_matvec fixtures: (type, rows=out, cols=in) at the microbenchmark shapes
MATVEC_CASES = [(t, r, c) for t in (Q8, Q5) for (r, c) in ((4096, 4096), (14336, 4096), (4096, 14336))]


def matvec_key(t, rows, cols):
    return f"y_{fwgpu.TYPE_NAMES[t]}_{rows}x{cols}"


def matvec_weights(t, rows, cols) -> np.ndarray:
    return fwgpu.synth_matrix(t, rows, cols, seed=1000 + 7 * t + rows + 3 * cols, scale_std=0.02)


def matvec_x(t, rows, cols) -> np.ndarray:
    return fwgpu.randn(2000 + t + cols, cols, 1.0)


# dequant fixtures: every code with a spread of fp16 scales incl. zero, subnormal, max
DEQUANT_SCALES = [0x0000, 0x8000, 0x0001, 0x0003, 0x01FF, 0x03FF, 0x8001, 0x0400, 0x3C00, 0xBC00,
                  0x2E66, 0x1A3F, 0x7BFF, 0xFBFF, 0x3555, 0x0A00]


def dequant_blocks(t) -> np.ndarray:
    bb = fwgpu.BLOCK_BYTES[t]
    rng = np.random.default_rng(100 + t)
    blocks = []
    for s in DEQUANT_SCALES:
        for k in range(8):
            b = np.zeros(bb, np.uint8)
            b[0], b[1] = s & 0xFF, s >> 8
            if t == Q8:
                b[2:] = (np.arange(32) + 32 * k).astype(np.uint8)          # all 256 codes
            else:
                b[2:] = rng.integers(0, 256, bb - 2).astype(np.uint8)
            blocks.append(b)
    return np.concatenate(blocks)


NORM_EPS = 1e-5
NORM_SIZES = [4, 288, 4096, 8192]


def norm_inputs(n):
    x = fwgpu.randn(300 + n, n, 1.0)
    w = (fwgpu.randn(400 + n, n, 0.01) + np.float32(1.0)).astype(np.float32)
    return x, w


ROPE_TABLES = [(64, 48, 10000.0), (64, 128, 500000.0), (16, 64, 10000.0)]
ROPE_CASES = [(0, 6, 48, 64, 10000.0, 0), (17, 6, 48, 64, 10000.0, 0), (63, 8, 128, 64, 500000.0, 0),
              (5, 2, 64, 16, 10000.0, 1)]


def rope_input(nh, hd):
    return fwgpu.randn(500 + nh * hd, nh * hd, 1.0)


def silu_input():
    x = fwgpu.randn(600, 4096, 3.0)
    special = np.array([0.0, -0.0, 1e-30, -1e-30, 1e-40, -1e-40, 88.0, -88.0, 89.0, -89.0, 100.0, -100.0,
                        20.0, -20.0, 1.0, -1.0, 0.5, -0.5, 3.4e38, -3.4e38], np.float32)
    return np.concatenate([special, x]).astype(np.float32)


DOT_SIZES = list(range(1, 68)) + [128, 288, 4096, 14336]


def dot_inputs(n):
    return fwgpu.randn(700 + n, n, 1.0), fwgpu.randn(800 + n, n, 1.0)


def argmax_cases():
    rng = np.random.default_rng(9)
    cases = [np.array([1, 2, 3, 4, 5], np.float32),
             np.array([5, 5, 5], np.float32),
             np.array([1, 7, 3, 7, 7, 2], np.float32),
             np.array([np.nan, 1, 2], np.float32),
             np.array([1, np.nan, 2, np.nan], np.float32),
             np.array([-np.inf, -np.inf], np.float32),
             np.array([-1.0, -0.0, 0.0, -0.5], np.float32),
             np.array([0.0, -0.0], np.float32),
             rng.standard_normal(32000).astype(np.float32),
             rng.standard_normal(128256).astype(np.float32)]
    big = rng.standard_normal(128256).astype(np.float32)
    big[[5, 90000, 128255]] = 9.0
    cases.append(big)
    return cases


# K-quant fixtures (kquant.npz): super-blocks of random bytes with the fp16 scale
# fields set from DEQUANT_SCALES (Q4_K: d and dmin; Q6_K: d), decoded by the
# reference's linear_get_row (linear.c:137-142 -> quant.c:87-188); quant_matvec
# outputs at these shapes (quant_matvec.c:231-261).
KQ_TYPES = (Q4K, Q6K)
KQ_MATVEC_CASES = [(Q4K, 4096, 4096), (Q4K, 4096, 14336), (Q6K, 4096, 4096), (Q6K, 1024, 4096)]


def kquant_blocks(t) -> np.ndarray:
    bb = fwgpu.BLOCK_BYTES[t]
    rng = np.random.default_rng(200 + t)
    blocks = []
    for i, s in enumerate(DEQUANT_SCALES):
        for k in range(2):
            b = rng.integers(0, 256, bb).astype(np.uint8)
            at = 208 if t == Q6K else 0
            b[at], b[at + 1] = s & 0xFF, s >> 8
            if t == Q4K:
                m = DEQUANT_SCALES[(i + 5 + k) % len(DEQUANT_SCALES)]
                b[2], b[3] = m & 0xFF, m >> 8
            blocks.append(b)
    return np.concatenate(blocks)


# sampler fixtures (sampler.npz): logits vectors x settings, one reference decision each
SAMPLE_SETTINGS = [(0.0, 0.9, 1.0), (0.0, 0.9, 1.3), (0.8, 0.9, 1.0), (0.8, 0.9, 1.1), (1.0, 1.0, 1.0),
                   (0.5, 0.5, 1.2), (1.5, 0.95, 1.05), (0.7, 0.2, 1.0)]
SAMPLE_SEEDS = [12345, 987654321, 2 ** 63 + 77]


def sample_cases():
    """(name, logits, hist) triples: spread-out, peaked, tied and large-vocabulary logits."""
    rng = np.random.default_rng(31)
    ties = rng.standard_normal(500).astype(np.float32)
    ties[100:140] = ties[3]                                       # equal probabilities
    peaked = (rng.standard_normal(4000) * 4.0).astype(np.float32)
    return [("n1000", rng.standard_normal(1000).astype(np.float32), rng.integers(0, 1000, 40).astype(np.uint32)),
            ("ties", ties, np.array([3, 3, 3, 7, 120, 499], np.uint32)),
            ("peaked", peaked, rng.integers(0, 4000, 200).astype(np.uint32)),
            ("v32000", rng.standard_normal(32000).astype(np.float32) * 2.0,
             rng.integers(0, 32000, 64).astype(np.uint32))]
