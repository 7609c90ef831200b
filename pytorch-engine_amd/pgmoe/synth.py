"""Seeded synthetic MoE layers in GGUF block form (benchmark and test inputs).

Draw order from ``np.random.default_rng(seed)`` is fixed: router weight -> (Zipf bias
permutation) -> gate, up, down expert blocks (expert-major) -> shared gate, up, down
blocks -> shared-expert input gate vector.  Activations come from an independent stream
``np.random.default_rng([seed, M])`` so the weights do not depend on how many tokens are
drawn.

Block contents follow the reference tests' random-block pattern
(tests/test_pygguf_engine.py:34-67): uniform random bytes with the fp16 super-block
scale(s) overwritten, here with d = |N(0,1)| * 0.02 * scale and dmin = |N(0,1)| * 0.01 * scale
(Q4_K / Q5_K / Q6_K) and Q8_0 blocks of d = |N(0,1)| * 0.01 * scale with int8 quants uniform in
[-127, 127].  ``scale=1`` is the benchmark scale; ``scale=0.01`` gives realistic GGUF
magnitudes where fp16 intermediates stay finite.
"""

from __future__ import annotations

from dataclasses import dataclass, field, replace
from typing import Dict, Optional, Tuple

import numpy as np

from .gguf import GGMLType, InMemoryGGUF, MoEConfig

Q4_0, Q4_1, Q5_0, Q4_K, Q5_K, Q6_K, Q8_0 = (GGMLType.Q4_0, GGMLType.Q4_1, GGMLType.Q5_0, GGMLType.Q4_K,
                                            GGMLType.Q5_K, GGMLType.Q6_K, GGMLType.Q8_0)

__all__ = ["LayerSpec", "CONFIGS", "SyntheticLayer", "DenseSpec", "DENSE_CONFIGS", "SyntheticDense",
           "random_blocks", "zipf_bias"]


@dataclass(frozen=True)
class LayerSpec:
    name: str
    hidden: int
    n_experts: int
    top_k: int
    inter: int
    qtypes: Tuple[int, int, int]  # gate, up, down
    norm_topk: bool = True
    arch: str = "qwen3moe"
    shared_inter: int = 0
    shared_qtypes: Tuple[int, int, int] = (Q8_0, Q8_0, Q8_0)
    shared_gate: bool = False
    zipf: bool = False  # harness-only router bias

    def expert_bytes(self) -> int:
        """GGUF bytes of one routed expert (gate + up + down)."""
        from .gguf import tensor_nbytes
        g = tensor_nbytes(self.qtypes[0], self.inter * self.hidden)
        u = tensor_nbytes(self.qtypes[1], self.inter * self.hidden)
        d = tensor_nbytes(self.qtypes[2], self.hidden * self.inter)
        return g + u + d

    def shared_bytes(self) -> int:
        from .gguf import tensor_nbytes
        if not self.shared_inter:
            return 0
        n = self.shared_inter * self.hidden
        return sum(tensor_nbytes(q, n) for q in self.shared_qtypes)


# BASELINE.json configs (C1..C5)
CONFIGS: Dict[str, LayerSpec] = {
    "tiny": LayerSpec("tiny", 1024, 8, 2, 512, (Q4_K, Q4_K, Q4_K)),
    "qwen3_30b_a3b": LayerSpec("qwen3_30b_a3b", 2048, 128, 8, 768, (Q4_K, Q4_K, Q6_K)),
    "qwen3_30b_a3b_zipf": LayerSpec("qwen3_30b_a3b_zipf", 2048, 128, 8, 768, (Q4_K, Q4_K, Q6_K),
                                    zipf=True),
    "mixtral_8x7b": LayerSpec("mixtral_8x7b", 4096, 8, 2, 14336, (Q4_K, Q4_K, Q4_K), arch="mixtral"),
    "qwen2_57b_a14b": LayerSpec("qwen2_57b_a14b", 3584, 64, 8, 2560, (Q8_0, Q8_0, Q8_0),
                                norm_topk=False, arch="qwen2moe", shared_inter=20480,
                                shared_gate=True),
}


def random_blocks(rng: np.random.Generator, qtype: int, rows: int, cols: int,
                  scale: float = 1.0) -> np.ndarray:
    """Raw GGUF bytes for a [rows, cols] matrix of random blocks (uint8, flat).  Float types
    (F32, F16, BF16): weights N(0, 1) * 0.02 * scale, in the type's own encoding (BF16: the
    fp32 value rounded to nearest even)."""
    if qtype in (GGMLType.F32, GGMLType.F16, GGMLType.BF16):
        f = (rng.standard_normal(rows * cols, dtype=np.float32) * np.float32(0.02 * scale)).astype(np.float32)
        if qtype == GGMLType.F32:
            return f.view(np.uint8)
        if qtype == GGMLType.F16:
            return f.astype(np.float16).view(np.uint8)
        u = f.view(np.uint32).astype(np.uint64)
        b16 = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)  # round to nearest even
        return b16.view(np.uint8)
    if qtype in (Q4_K, Q5_K):
        nb = rows * (cols // 256)
        raw = rng.integers(0, 256, size=(nb, 144 if qtype == Q4_K else 176), dtype=np.uint8)
        d = (np.abs(rng.standard_normal(nb)) * (0.02 * scale)).astype(np.float16)
        dmin = (np.abs(rng.standard_normal(nb)) * (0.01 * scale)).astype(np.float16)
        raw[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        raw[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
    elif qtype == Q6_K:
        nb = rows * (cols // 256)
        raw = rng.integers(0, 256, size=(nb, 210), dtype=np.uint8)
        d = (np.abs(rng.standard_normal(nb)) * (0.02 * scale)).astype(np.float16)
        raw[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    elif qtype == Q5_0:
        nb = rows * (cols // 32)
        raw = rng.integers(0, 256, size=(nb, 22), dtype=np.uint8)
        d = (np.abs(rng.standard_normal(nb)) * (0.02 * scale)).astype(np.float16)
        raw[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    elif qtype == Q4_1:  # d = |N| * 0.02 scale, m = -N(0, 1) * 0.1 scale (centres the codes)
        nb = rows * (cols // 32)
        raw = rng.integers(0, 256, size=(nb, 20), dtype=np.uint8)
        d = (np.abs(rng.standard_normal(nb)) * (0.02 * scale)).astype(np.float16)
        m = (-np.abs(rng.standard_normal(nb)) * (0.1 * scale)).astype(np.float16)
        raw[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        raw[:, 2:4] = m.view(np.uint8).reshape(nb, 2)
    elif qtype == GGMLType.Q5_1:  # d = |N| * 0.01 scale, m = -N(0, 1) * 0.15 scale (centres the 5-bit codes)
        nb = rows * (cols // 32)
        raw = rng.integers(0, 256, size=(nb, 24), dtype=np.uint8)
        d = (np.abs(rng.standard_normal(nb)) * (0.01 * scale)).astype(np.float16)
        m = (-np.abs(rng.standard_normal(nb)) * (0.15 * scale)).astype(np.float16)
        raw[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        raw[:, 2:4] = m.view(np.uint8).reshape(nb, 2)
    elif qtype == Q4_0:
        nb = rows * (cols // 32)
        raw = rng.integers(0, 256, size=(nb, 18), dtype=np.uint8)
        d = (np.abs(rng.standard_normal(nb)) * (0.02 * scale)).astype(np.float16)
        raw[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    elif qtype == Q8_0:
        nb = rows * (cols // 32)
        raw = np.empty((nb, 34), dtype=np.uint8)
        d = (np.abs(rng.standard_normal(nb)) * (0.01 * scale)).astype(np.float16)
        raw[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        raw[:, 2:34] = rng.integers(-127, 128, size=(nb, 32), dtype=np.int8).view(np.uint8)
    elif qtype in (GGMLType.Q2_K, GGMLType.Q3_K, GGMLType.IQ4_XS):
        # random bytes; the fp16 d (and Q2_K's dmin) small: Q2_K d |N| * 0.02 scale, dmin
        # |N| * 0.01 scale; Q3_K d |N| * 0.02 scale; IQ4_XS d |N| * 0.001 scale (its sub-block
        # scales reach 32 and its levels 127)
        nbytes = {GGMLType.Q2_K: 84, GGMLType.Q3_K: 110, GGMLType.IQ4_XS: 136}[qtype]
        nb = rows * (cols // 256)
        raw = rng.integers(0, 256, size=(nb, nbytes), dtype=np.uint8)
        dscale = 0.001 if qtype == GGMLType.IQ4_XS else 0.02
        d = (np.abs(rng.standard_normal(nb)) * (dscale * scale)).astype(np.float16).view(np.uint8).reshape(nb, 2)
        if qtype == GGMLType.Q2_K:
            raw[:, 80:82] = d
            raw[:, 82:84] = (np.abs(rng.standard_normal(nb)) * (0.01 * scale)).astype(np.float16).view(
                np.uint8).reshape(nb, 2)
        elif qtype == GGMLType.Q3_K:
            raw[:, 108:110] = d
        else:
            raw[:, 0:2] = d
    elif qtype == GGMLType.IQ4_NL:  # d = |N| * 0.01 scale (levels up to 127)
        nb = rows * (cols // 32)
        raw = rng.integers(0, 256, size=(nb, 18), dtype=np.uint8)
        raw[:, 0:2] = (np.abs(rng.standard_normal(nb)) * (0.01 * scale)).astype(np.float16).view(np.uint8).reshape(nb, 2)
    elif qtype == GGMLType.MXFP4:  # exponent byte 118..123: block scales 2^-10 .. 2^-5 (times scale's power of 2)
        nb = rows * (cols // 32)
        raw = rng.integers(0, 256, size=(nb, 17), dtype=np.uint8)
        shift = int(np.round(np.log2(scale))) if scale > 0 else 0
        raw[:, 0] = np.clip(rng.integers(118, 124, size=nb) + shift, 0, 255).astype(np.uint8)
    else:
        raise ValueError(f"unsupported qtype {qtype}")
    return raw.reshape(-1)


def zipf_bias(rng: np.random.Generator, n_experts: int, s: float = 1.1) -> np.ndarray:
    """bias[e] = log ZipfPMF_s(rank_e) over a random expert permutation (fp32)."""
    perm = rng.permutation(n_experts)
    ranks = np.arange(1, n_experts + 1, dtype=np.float64)
    pmf = ranks ** (-s) / np.sum(ranks ** (-s))
    return np.log(pmf[perm]).astype(np.float32)


@dataclass
class SyntheticLayer:
    """One seeded MoE layer exposed through the GGUF reader surface (layer index 0)."""

    spec: LayerSpec
    seed: int = 0
    scale: float = 1.0
    gguf: InMemoryGGUF = field(init=False)
    config: MoEConfig = field(init=False)
    router_bias: Optional[np.ndarray] = field(init=False, default=None)

    def __post_init__(self) -> None:
        sp = self.spec
        rng = np.random.default_rng(self.seed)
        meta = {
            "general.architecture": sp.arch,
            f"{sp.arch}.embedding_length": sp.hidden,
            f"{sp.arch}.expert_count": sp.n_experts,
            f"{sp.arch}.expert_used_count": sp.top_k,
            f"{sp.arch}.expert_feed_forward_length": sp.inter,
            f"{sp.arch}.expert_weights_norm": sp.norm_topk,
        }
        if sp.shared_inter:
            meta[f"{sp.arch}.expert_shared_feed_forward_length"] = sp.shared_inter
        g = InMemoryGGUF(meta)
        H, E, I = sp.hidden, sp.n_experts, sp.inter
        router = (rng.standard_normal((E, H), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
        g.add_tensor("blk.0.ffn_gate_inp.weight", (E, H), GGMLType.F32, router.view(np.uint8))
        if sp.zipf:
            self.router_bias = zipf_bias(rng, E)
        shapes = {"gate": (I, H), "up": (I, H), "down": (H, I)}
        for qt, proj in zip(sp.qtypes, ("gate", "up", "down")):
            n, k = shapes[proj]
            raw = np.concatenate([random_blocks(rng, qt, n, k, self.scale) for _ in range(E)])
            g.add_tensor(f"blk.0.ffn_{proj}_exps.weight", (E, n, k), qt, raw)
        if sp.shared_inter:
            Is = sp.shared_inter
            sshapes = {"gate": (Is, H), "up": (Is, H), "down": (H, Is)}
            for qt, proj in zip(sp.shared_qtypes, ("gate", "up", "down")):
                n, k = sshapes[proj]
                g.add_tensor(f"blk.0.ffn_{proj}_shexp.weight", (n, k), qt,
                             random_blocks(rng, qt, n, k, self.scale))
            if sp.shared_gate:
                gv = (rng.standard_normal(H, dtype=np.float32) * np.float32(0.02)).astype(np.float32)
                g.add_tensor("blk.0.ffn_gate_inp_shexp.weight", (H,), GGMLType.F32, gv.view(np.uint8))
        self.gguf = g
        self.config = g.build_model_config()

    def draw_x(self, M: int) -> np.ndarray:
        """fp16 activations [M, hidden] ~ N(0, 1)."""
        rng = np.random.default_rng([self.seed, M])
        return rng.standard_normal((M, self.spec.hidden), dtype=np.float32).astype(np.float16)

    def tensor(self, name: str) -> np.ndarray:
        return self.gguf.get_tensor_bytes(f"blk.0.{name}")


def with_shape(spec: LayerSpec, **kw) -> LayerSpec:
    """A copy of ``spec`` with some fields replaced (smaller test layers)."""
    return replace(spec, **kw)


# ---------------------------------------------------------------- dense SwiGLU FFN
@dataclass(frozen=True)
class DenseSpec:
    name: str
    hidden: int
    inter: int
    qtypes: Tuple[int, int, int]  # gate, up, down
    arch: str = "qwen3"

    def weight_bytes(self) -> int:
        from .gguf import tensor_nbytes
        n = self.inter * self.hidden
        return sum(tensor_nbytes(q, n) for q in self.qtypes)


# Dense FFN shapes (the reference's GGUFDenseMLP, model.py:778-846): a small one for tests,
# an 8B-class Q4_K_M layer (gate/up Q4_K, down Q6_K) and an all-Q8_0 one.
DENSE_CONFIGS: Dict[str, DenseSpec] = {
    "dense_tiny": DenseSpec("dense_tiny", 1024, 2816, (Q4_K, Q4_K, Q6_K)),
    "dense_q8": DenseSpec("dense_q8", 2048, 5632, (Q8_0, Q8_0, Q8_0), arch="llama"),
    "dense_8b": DenseSpec("dense_8b", 4096, 12288, (Q4_K, Q4_K, Q6_K)),
}


@dataclass
class SyntheticDense:
    """One seeded dense FFN (blk.0.ffn_{gate,up,down}.weight) through the GGUF reader surface."""

    spec: DenseSpec
    seed: int = 0
    scale: float = 1.0
    gguf: InMemoryGGUF = field(init=False)
    config: MoEConfig = field(init=False)

    def __post_init__(self) -> None:
        sp = self.spec
        rng = np.random.default_rng([self.seed, 7])
        g = InMemoryGGUF({"general.architecture": sp.arch, f"{sp.arch}.embedding_length": sp.hidden,
                          f"{sp.arch}.feed_forward_length": sp.inter})
        H, I = sp.hidden, sp.inter
        shapes = {"gate": (I, H), "up": (I, H), "down": (H, I)}
        for qt, proj in zip(sp.qtypes, ("gate", "up", "down")):
            n, k = shapes[proj]
            g.add_tensor(f"blk.0.ffn_{proj}.weight", (n, k), qt, random_blocks(rng, qt, n, k, self.scale))
        self.gguf = g
        self.config = g.build_model_config()

    def draw_x(self, M: int) -> np.ndarray:
        """fp16 activations [M, hidden] ~ N(0, 1)."""
        rng = np.random.default_rng([self.seed, M, 7])
        return rng.standard_normal((M, self.spec.hidden), dtype=np.float32).astype(np.float16)

    def tensor(self, name: str) -> np.ndarray:
        return self.gguf.get_tensor_bytes(f"blk.0.{name}")
