"""Decode-step projection chain: the quantised matmuls of
one decode step of a 28-layer Qwen3-0.6B-shaped model in a Q4_K_M mix.

Per layer (Gemma4LanguageModel.encodeProjection order,
Sources/EdgeRunner/Models/Gemma4LanguageModel.swift:2036-2246, 3465-3580,
4207-4285; Llama decode pass LlamaLanguageModel.swift:4308-4528):

    q    2048 x 1024  Q4_K      <- h  (hidden, 1024)
    k    1024 x 1024  Q4_K      <- h
    v    1024 x 1024  Q4_K      <- h
    o    1024 x 2048  Q4_K      <- a  (attention output, 2048)
    gate 3072 x 1024  Q4_K      <- h
    up   3072 x 1024  Q4_K      <- h
    down 1024 x 3072  Q6_K      <- f  (gated activation, 3072)
then the LM head 151936 x 1024 Q6_K <- h.

The non-matmul operations between them (norms, RoPE, attention, the gated
activation, residual adds) are not part of this path, so every projection
reads a fixed activation vector of its input width ("hidden state re-used as
is"); the encodes still go onto one stream in decode-step order, so each
launch waits for the previous one exactly as in a decode step.

Two execution forms are recorded into a HIP graph:
  * per-projection: 7 launches per layer + head = 197 (the reference's
    dispatch pattern);
  * fused: q/k/v as one triple projection and gate/up as one dual projection
    (encodeQ4KWeightsTriple / encodeQ4KWeightsDual, one x read each),
    4 launches per layer + head = 113.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import numpy as np

from . import synth
from .gemv import GEMVKernel
from .runtime import Buffer, Capture, Context, Graph, Stream

BLOCK = {"q4_k": (144, 256), "q6_k": (210, 256), "q8_0": (34, 32)}
DSCALE = {"q8_0": {"dscale": 0.02}, "q4_k": {"dscale": 0.01, "dminscale": 0.01},
          "q6_k": {"dscale": 0.005}}


@dataclass
class ChainSpec:
    layers: int = 28
    hidden: int = 1024
    q_dim: int = 2048
    kv_dim: int = 1024
    ffn: int = 3072
    vocab: int = 151936
    attn_fmt: str = "q4_k"
    up_fmt: str = "q4_k"
    down_fmt: str = "q6_k"
    head_fmt: str = "q6_k"

    def layer_projections(self) -> List[Tuple[str, str, int, int, str]]:
        """(name, format, rows M, columns K, input vector)"""
        return [("q", self.attn_fmt, self.q_dim, self.hidden, "h"),
                ("k", self.attn_fmt, self.kv_dim, self.hidden, "h"),
                ("v", self.attn_fmt, self.kv_dim, self.hidden, "h"),
                ("o", self.attn_fmt, self.hidden, self.q_dim, "a"),
                ("gate", self.up_fmt, self.ffn, self.hidden, "h"),
                ("up", self.up_fmt, self.ffn, self.hidden, "h"),
                ("down", self.down_fmt, self.hidden, self.ffn, "f")]

    def all_projections(self) -> List[Tuple[Tuple[int, str], str, int, int, str]]:
        out = [((l, n), f, M, K, src) for l in range(self.layers)
               for n, f, M, K, src in self.layer_projections()]
        out.append(((-1, "head"), self.head_fmt, self.vocab, self.hidden, "h"))
        return out

    def weight_bytes(self) -> int:
        tot = 0
        for _, f, M, K, _ in self.all_projections():
            bb, bw = BLOCK[f]
            tot += M * (K // bw) * bb
        return tot

    def launches(self, fused: bool) -> int:
        return self.layers * (4 if fused else 7) + 1


def make_weights(spec: ChainSpec, config: int = 5) -> Dict[Tuple[int, str], np.ndarray]:
    """Seeded synthetic weights, BASELINE distributions per format; tensor t of
    the chain uses seed(config, 16 + t)."""
    ws = {}
    for t, (key, f, M, K, _) in enumerate(spec.all_projections()):
        ws[key] = synth.weights(f, synth.seed(config, 16 + t), M, K, **DSCALE[f])
    return ws


def make_inputs(spec: ChainSpec, config: int = 5) -> Dict[str, np.ndarray]:
    return {"h": synth.normal_f32(synth.seed(config, 1), spec.hidden),
            "a": synth.normal_f32(synth.seed(config, 2), spec.q_dim),
            "f": synth.normal_f32(synth.seed(config, 3), spec.ffn)}


class DecodeChain:
    """Device-resident weights, inputs and outputs of one decode step's
    projections, encoded onto a stream or recorded into a graph."""

    def __init__(self, ctx: Context, spec: ChainSpec, weights: Dict[Tuple[int, str], np.ndarray],
                 inputs: Dict[str, np.ndarray], stream: Optional[Stream] = None):
        self.ctx, self.spec = ctx, spec
        self.gemv = GEMVKernel(ctx)
        self.w: Dict[Tuple[int, str], Buffer] = {k: ctx.upload(v, stream) for k, v in weights.items()}
        self.x: Dict[str, Buffer] = {k: ctx.upload(v, stream) for k, v in inputs.items()}
        self.y: Dict[Tuple[int, str], Buffer] = {
            key: ctx.alloc(4 * M) for key, _, M, _, _ in spec.all_projections()}
        self.meta = {key: (f, M, K, src) for key, f, M, K, src in spec.all_projections()}

    def _single(self, stream, key):
        f, M, K, src = self.meta[key]
        enc = {"q4_k": self.gemv.encodeQ4KWeights, "q6_k": self.gemv.encodeQ6KWeights,
               "q8_0": self.gemv.encodeQ8_0Weights}[f]
        enc(stream, self.w[key], self.x[src], self.y[key], M, K)

    def encode(self, stream: Stream, fused: bool = False) -> None:
        s = self.spec
        for l in range(s.layers):
            if fused and s.attn_fmt == "q4_k":
                self.gemv.encodeQ4KWeightsTriple(
                    stream, self.w[(l, "q")], self.w[(l, "k")], self.w[(l, "v")], self.x["h"],
                    self.y[(l, "q")], self.y[(l, "k")], self.y[(l, "v")], s.q_dim, s.kv_dim,
                    s.kv_dim, s.hidden)
            else:
                for n in ("q", "k", "v"):
                    self._single(stream, (l, n))
            self._single(stream, (l, "o"))
            if fused and s.up_fmt == "q4_k":
                self.gemv.encodeQ4KWeightsDual(
                    stream, self.w[(l, "gate")], self.w[(l, "up")], self.x["h"],
                    self.y[(l, "gate")], self.y[(l, "up")], s.ffn, s.hidden)
            else:
                for n in ("gate", "up"):
                    self._single(stream, (l, n))
            self._single(stream, (l, "down"))
        self._single(stream, (-1, "head"))

    def capture(self, stream: Stream, fused: bool = False) -> Graph:
        with Capture(self.ctx, stream) as cap:
            self.encode(stream, fused)
        return cap.graph

    def outputs(self, stream: Optional[Stream] = None) -> Dict[Tuple[int, str], np.ndarray]:
        return {k: b.download(np.float32, stream=stream) for k, b in self.y.items()}

    def free(self) -> None:
        for d in (self.w, self.x, self.y):
            for b in d.values():
                b.free()
