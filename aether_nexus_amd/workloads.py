"""Seeded synthetic Weaver decode workloads.

Shapes follow the reference's pools (nexus-core/src/fabric.rs:124-186,
weaver_kernel.metal:110-117): hot pool ``[blocks][16][kv_heads][head_dim]`` f16,
cold pool ``[blocks][16][kv_heads]`` SparseCodes, block tables of hot refs then
cold refs per sequence, dictionary ``[dict_heads][atoms][head_dim]`` f16.  Every
sequence owns its own physical blocks, assigned through a seeded permutation so
the block table is exercised.  Tensors are generated with torch on any device
(identical code for host-side parity cases and device-side benchmark pools).

Named workloads (sizes in tokens; "cold" counts codes per kv head):
  tiny         8 q / 8 kv heads, d 64, hot 256, cold 1024, 512 atoms, scale 1 with q ~ N(0,1)/8
  hot_only     32 q / 8 kv, d 128, hot 4096, no cold, scale 1/sqrt(128)
  hot_cold     32 / 8 / 128, hot 2048, cold 32768, 4096 atoms shared, scale 1/sqrt(128)
  batched      batch 64, hot 1024, cold 131072, Zipf(1.1) atom indices
  spec_verify  32 layers, batch 8, 8 causal draft queries, hot 2048, cold 65536, per-layer dictionary
  sweep(B)     hot_cold at batch B
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field, replace
from typing import Optional

import numpy as np
import torch

from .types import BLOCK_SIZE


@dataclass(frozen=True)
class Geometry:
    layers: int = 1
    batch: int = 1
    queries: int = 1
    q_heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    dict_size: int = 4096
    dict_heads: int = 1          # 1 = one shared dictionary, kv_heads = per-kv-head (reference)
    hot_count: int = 0           # blocks of 16 tokens per sequence
    cold_count: int = 0
    scale: float = 1.0
    causal: bool = False
    separate_v: bool = False
    q_std: float = 1.0
    coef_std: float = 0.5
    zipf: Optional[float] = None  # None = uniform atom indices
    copies: int = 1               # disjoint block sets (bench rotation)
    tag_bit31: bool = False       # set bit 31 on every other ref (masked by the kernel)

    @property
    def gqa(self) -> int:
        return self.q_heads // self.kv_heads

    @property
    def rows_r(self) -> int:
        return self.gqa * self.queries

    @property
    def refs_stride(self) -> int:
        return self.hot_count + self.cold_count

    @property
    def hot_blocks(self) -> int:
        return self.copies * self.batch * self.hot_count

    @property
    def cold_blocks(self) -> int:
        return self.copies * self.batch * self.cold_count

    @property
    def tokens(self) -> int:
        """Query tokens decoded per step (B*Q); layers do not add tokens."""
        return self.batch * self.queries

    def algorithmic_bytes(self) -> dict:
        """Compulsory HBM bytes of one decode step, by part (intermediates excluded):
        hot K(=V) rows, cold codes, dictionary, q in + out, block refs."""
        L, B, Q = self.layers, self.batch, self.queries
        nh, nc = self.hot_count * BLOCK_SIZE, self.cold_count * BLOCK_SIZE
        kv_tensors = 2 if self.separate_v else 1
        hot = L * B * nh * self.kv_heads * self.head_dim * 2 * kv_tensors
        cold = L * B * nc * self.kv_heads * 16
        dic = L * self.dict_size * self.head_dim * 2 * self.dict_heads if self.cold_count else 0
        qo = L * 2 * B * Q * self.q_heads * self.head_dim * 2
        refs = L * B * (self.hot_count + self.cold_count) * 4
        return {"hot": hot, "cold": cold, "dict": dic, "q_out": qo, "refs": refs,
                "total": hot + cold + dic + qo + refs}

    def proj_flops(self) -> int:
        if not self.cold_count:
            return 0
        return 2 * self.layers * self.batch * self.queries * self.q_heads * self.dict_size * self.head_dim


def tiny(**kw) -> Geometry:
    return replace(Geometry(q_heads=8, kv_heads=8, head_dim=64, dict_size=512, hot_count=16, cold_count=64,
                            scale=1.0, q_std=1.0 / 8.0), **kw)


def hot_only(**kw) -> Geometry:
    return replace(Geometry(hot_count=256, cold_count=0, dict_size=0, scale=1.0 / math.sqrt(128)), **kw)


def hot_cold(**kw) -> Geometry:
    return replace(Geometry(hot_count=128, cold_count=2048, dict_size=4096, scale=1.0 / math.sqrt(128)), **kw)


def batched(**kw) -> Geometry:
    return replace(Geometry(batch=64, hot_count=64, cold_count=8192, dict_size=4096, scale=1.0 / math.sqrt(128),
                            zipf=1.1), **kw)


def spec_verify(**kw) -> Geometry:
    return replace(Geometry(layers=32, batch=8, queries=8, hot_count=128, cold_count=4096, dict_size=4096,
                            scale=1.0 / math.sqrt(128), causal=True), **kw)


def sweep(batch: int, **kw) -> Geometry:
    return hot_cold(batch=batch, **kw)


NAMED = {"tiny": tiny, "hot_only": hot_only, "hot_cold": hot_cold, "batched": batched,
         "spec_verify": spec_verify}


@dataclass
class Workload:
    """Inputs of one decode request.  f16 tensors are torch.float16; codes are
    int16 words ``[..., 8]`` (4 u16 indices then 4 f16 coefficient bit patterns);
    refs are int32 holding the u32 block refs."""

    geom: Geometry
    q: torch.Tensor
    hot_k: Optional[torch.Tensor]
    hot_v: Optional[torch.Tensor]
    cold: Optional[torch.Tensor]
    refs: torch.Tensor          # [copies][L][B][refs_stride]
    dictionary: Optional[torch.Tensor]
    q_latent: Optional[torch.Tensor] = None
    seq_hot: Optional[torch.Tensor] = None
    seq_cold: Optional[torch.Tensor] = None
    extra: dict = field(default_factory=dict)

    def out_shape(self) -> tuple:
        g = self.geom
        return (g.layers, g.batch, g.queries, g.q_heads, g.head_dim)

    def to(self, device) -> "Workload":
        def mv(t):
            return None if t is None else t.to(device)
        return Workload(self.geom, mv(self.q), mv(self.hot_k), mv(self.hot_v), mv(self.cold), mv(self.refs),
                        mv(self.dictionary), mv(self.q_latent), mv(self.seq_hot), mv(self.seq_cold),
                        dict(self.extra))


def _zipf_ranks(gen: torch.Generator, n: int, atoms: int, s: float, device) -> torch.Tensor:
    k = torch.arange(1, atoms + 1, dtype=torch.float64, device=device)
    cdf = torch.cumsum(k.pow(-s), 0)
    cdf = cdf / cdf[-1]
    out = torch.empty(n, dtype=torch.int64, device=device)
    chunk = 1 << 24
    for i in range(0, n, chunk):
        m = min(chunk, n - i)
        u = torch.rand(m, generator=gen, dtype=torch.float64, device=device)
        out[i:i + m] = torch.clamp(torch.searchsorted(cdf, u, right=True), max=atoms - 1)
    return out


def make_codes(gen: torch.Generator, shape: tuple, atoms: int, coef_std: float, zipf: Optional[float],
               device) -> torch.Tensor:
    """SparseCode words int16 [*shape, 8]: indices uniform over atoms (or Zipf(s)
    ranks mapped through a seeded permutation), coefficients ~ N(0, coef_std)."""
    n = int(np.prod(shape)) * 4
    if zipf is None:
        idx = torch.randint(0, atoms, (n,), generator=gen, device=device, dtype=torch.int64)
    else:
        perm = torch.randperm(atoms, generator=gen, device=device)
        idx = perm[_zipf_ranks(gen, n, atoms, zipf, device)]
    coef = (torch.randn(n, generator=gen, device=device, dtype=torch.float32) * coef_std).to(torch.float16)
    idx16 = torch.where(idx >= 32768, idx - 65536, idx).to(torch.int16)
    words = torch.empty(tuple(shape) + (8,), dtype=torch.int16, device=device)
    words[..., :4] = idx16.view(tuple(shape) + (4,))
    words[..., 4:] = coef.view(torch.int16).view(tuple(shape) + (4,))
    return words


def generate(geom: Geometry, seed: int = 0, device="cpu") -> Workload:
    """Seeded inputs for ``geom`` on ``device``."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    L, B, Q, Hq, Hkv, D = geom.layers, geom.batch, geom.queries, geom.q_heads, geom.kv_heads, geom.head_dim
    q = (torch.randn((L, B, Q, Hq, D), generator=gen, device=device) * geom.q_std).to(torch.float16)
    hot_k = hot_v = cold = dictionary = None
    if geom.hot_count:
        hot_k = torch.randn((L, geom.hot_blocks, BLOCK_SIZE, Hkv, D), generator=gen, device=device,
                            dtype=torch.float32).to(torch.float16)
        if geom.separate_v:
            hot_v = torch.randn(hot_k.shape, generator=gen, device=device, dtype=torch.float32).to(torch.float16)
    if geom.cold_count:
        cold = make_codes(gen, (L, geom.cold_blocks, BLOCK_SIZE, Hkv), geom.dict_size, geom.coef_std, geom.zipf,
                          device)
        dd = torch.randn((L, geom.dict_heads, geom.dict_size, D), generator=gen, device=device,
                         dtype=torch.float64)
        dictionary = (dd / dd.norm(dim=-1, keepdim=True)).to(torch.float16)
    # Block tables: copy c, layer l, sequence b own blocks [(c*B + b)*count, +count) of a permutation.
    refs = torch.zeros((geom.copies, L, B, max(geom.refs_stride, 1)), dtype=torch.int64, device=device)
    for l in range(L):
        if geom.hot_count:
            perm = torch.randperm(geom.hot_blocks, generator=gen, device=device)
            refs[:, l, :, :geom.hot_count] = perm.view(geom.copies, B, geom.hot_count)
        if geom.cold_count:
            perm = torch.randperm(geom.cold_blocks, generator=gen, device=device)
            refs[:, l, :, geom.hot_count:geom.refs_stride] = perm.view(geom.copies, B, geom.cold_count)
    if geom.tag_bit31:
        tag = torch.zeros_like(refs)
        tag[..., 1::2] = 1 << 31
        refs = refs | tag
    refs32 = torch.where(refs >= 2 ** 31, refs - 2 ** 32, refs).to(torch.int32)
    return Workload(geom, q, hot_k, hot_v, cold, refs32, dictionary)


# ------------------------------------------------------------ host views


def host_arrays(wl: Workload, copy: int = 0) -> dict:
    """numpy views for the oracle: f16 tensors as uint16 bits, codes as uint16
    words [..., 8], refs of one copy as uint32."""
    def bits(t):
        if t is None:
            return None
        t = t.detach().to("cpu").contiguous()
        if t.dtype == torch.float16:
            return t.view(torch.int16).numpy().view(np.uint16)
        if t.dtype == torch.int16:
            return t.numpy().view(np.uint16)
        raise TypeError(t.dtype)
    refs = wl.refs[copy].detach().to("cpu").contiguous().numpy().view(np.uint32)
    out = {"q": bits(wl.q), "hot_k": bits(wl.hot_k), "hot_v": bits(wl.hot_v), "cold": bits(wl.cold),
           "refs": refs, "dictionary": bits(wl.dictionary), "q_latent": bits(wl.q_latent)}
    for k in ("seq_hot", "seq_cold"):
        t = getattr(wl, k)
        out[k] = None if t is None else t.detach().to("cpu").contiguous().numpy().view(np.uint32)
    return out


def head_blocked(cold: torch.Tensor) -> torch.Tensor:
    """The cold pool [L][blocks][16][kv_heads][8] reordered to
    [L][blocks][kv_heads][16][8] (AW_F_COLD_HEAD_BLOCKED)."""
    return cold.permute(0, 1, 3, 2, 4).contiguous()


def device_desc(wl: Workload, out: torch.Tensor, copy: int = 0, cold_head_blocked: Optional[torch.Tensor] = None,
                q_latent_f32: bool = False):
    """``aw_decode_desc`` for a workload whose tensors live on the GPU.
    ``cold_head_blocked``: the workload's cold pool reordered by head_blocked();
    the descriptor then points at it and sets AW_F_COLD_HEAD_BLOCKED.
    ``q_latent_f32``: a q_latent computed on the device stays fp32."""
    from .weaver import make_desc
    g = wl.geom
    return make_desc(layers=g.layers, batch=g.batch, queries=g.queries, q_heads=g.q_heads, kv_heads=g.kv_heads,
                     head_dim=g.head_dim, dict_size=g.dict_size, dict_heads=g.dict_heads, hot_count=g.hot_count,
                     cold_count=g.cold_count, refs_stride=max(g.refs_stride, 1), hot_blocks=g.hot_blocks,
                     cold_blocks=g.cold_blocks, q=wl.q, out=out, hot_k=wl.hot_k, hot_v=wl.hot_v,
                     cold=wl.cold if cold_head_blocked is None else cold_head_blocked,
                     refs=wl.refs[copy], dictionary=wl.dictionary, q_latent=wl.q_latent, seq_hot=wl.seq_hot,
                     seq_cold=wl.seq_cold, scale=g.scale, causal=g.causal,
                     cold_head_blocked=cold_head_blocked is not None, q_latent_f32=q_latent_f32)
