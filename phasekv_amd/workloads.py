"""Seeded synthetic workloads of the benchmark configurations.

Dense fp16 K/V are generated on the host with ``torch.Generator().manual_seed``
(so any consumer can regenerate identical bits), copied to the device and
packed there by the HIP ``quantize_pack``.

Configs (group size 32 everywhere):

* C1  Qwen2.5-0.5B shape: B1, Hq14, Hkv2, hd64; prompt 512 @4-bit, no cold, hot 32.
* C2  Qwen2.5-7B shape:   B1, Hq28, Hkv4, hd128; prompt 4096 @2-bit, cold 256 @4-bit,
      hot 128; K ~ N(0,1) with 4 outlier channels per kv head scaled x8.
* C3  C2 shape with prompt 4096/8192/16384/32768 @2-bit, cold 512 @4-bit, hot 128.
* C4  batch 16, prompt rows ragged in [4096, 8192] @4-bit, cold 1024 @2-bit, hot 64.
* C5  Llama-3-8B shape: B8, Hq32, Hkv8, hd128; prompt 16384 @2-bit, cold 2048 @8-bit,
      hot 256; K ~ Student-t(df=3).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional

import numpy as np
import torch

from .tiers import LayerTiers, PackedKVSegment, pack_kv

GROUP = 32


@dataclass(frozen=True)
class Config:
    name: str
    batch: int
    hq: int
    hkv: int
    hd: int
    prompt: int
    prompt_bits: int
    cold: int
    cold_bits: int
    hot: int
    k_kind: str = "normal"        # normal | outliers | student_t
    ragged_min: int = 0           # > 0: prompt rows have lengths in [ragged_min, prompt]

    @property
    def tokens(self) -> int:
        return self.prompt + self.cold + self.hot


CONFIGS = {
    "C1": Config("C1", 1, 14, 2, 64, 512, 4, 0, 4, 32),
    "C2": Config("C2", 1, 28, 4, 128, 4096, 2, 256, 4, 128, "outliers"),
    "C3-4K": Config("C3-4K", 1, 28, 4, 128, 4096, 2, 512, 4, 128, "outliers"),
    "C3-8K": Config("C3-8K", 1, 28, 4, 128, 8192, 2, 512, 4, 128, "outliers"),
    "C3-16K": Config("C3-16K", 1, 28, 4, 128, 16384, 2, 512, 4, 128, "outliers"),
    "C3-32K": Config("C3-32K", 1, 28, 4, 128, 32768, 2, 512, 4, 128, "outliers"),
    "C4": Config("C4", 16, 28, 4, 128, 8192, 4, 1024, 2, 64, "normal", 4096),
    "C5": Config("C5", 8, 32, 8, 128, 16384, 2, 2048, 8, 256, "student_t"),
}


def _packed_bytes(tokens: int, hd: int, bits: int, gs: int = GROUP) -> int:
    """Algorithmic bytes of one kv head's packed K+V for ``tokens`` tokens (codes + fp16 meta)."""
    vpb = 8 // bits
    k = hd * -(-tokens // vpb) + 4 * hd * -(-tokens // min(gs, tokens))
    v = tokens * -(-hd // vpb) + 4 * tokens * -(-hd // min(gs, hd))
    return k + v


def algorithmic_bytes(cfg: Config, prompt_lens: Optional[List[int]] = None) -> int:
    """HBM bytes one decode step must move: packed tiers + fp16 hot + q + output.

    Split partials are excluded (reported separately).
    """
    total = 0
    lens = prompt_lens if prompt_lens is not None else [cfg.prompt] * cfg.batch
    for b in range(cfg.batch):
        per_head = _packed_bytes(lens[b], cfg.hd, cfg.prompt_bits)
        if cfg.cold:
            per_head += _packed_bytes(cfg.cold, cfg.hd, cfg.cold_bits)
        per_head += 4 * cfg.hd * cfg.hot
        total += per_head * cfg.hkv
    total += 2 * 2 * cfg.batch * cfg.hq * cfg.hd
    return total


def fp16_dense_bytes(cfg: Config, prompt_lens: Optional[List[int]] = None) -> int:
    """Bytes of the FP16 dense comparator over the same tokens."""
    lens = prompt_lens if prompt_lens is not None else [cfg.prompt] * cfg.batch
    toks = sum(l + cfg.cold + cfg.hot for l in lens)
    return toks * cfg.hkv * 4 * cfg.hd + 2 * 2 * cfg.batch * cfg.hq * cfg.hd


def _dense(gen: torch.Generator, shape, kind: str, seed: int) -> torch.Tensor:
    if kind == "student_t":
        rng = np.random.default_rng(seed)
        return torch.from_numpy(rng.standard_t(3, size=shape).astype(np.float32)).to(torch.float16)
    x = torch.randn(*shape, generator=gen, dtype=torch.float32)
    if kind == "outliers":
        hd = shape[-1]
        for h in range(shape[1]):
            ch = torch.randperm(hd, generator=gen)[:4]
            x[:, h, :, ch] *= 8.0
    return x.to(torch.float16)


@dataclass
class Workload:
    cfg: Config
    q: torch.Tensor                 # [B, Hq, hd] fp16 on the device
    tiers: LayerTiers
    prompt_lens: Optional[torch.Tensor]   # int32 [B] on the device, ragged configs only
    prompt_lens_list: List[int]
    dense_k: Optional[List[torch.Tensor]] = None   # host fp16 per tier (prompt, cold, hot)
    dense_v: Optional[List[torch.Tensor]] = None

    @property
    def bytes(self) -> int:
        return algorithmic_bytes(self.cfg, self.prompt_lens_list)


def make_workload(cfg: Config, device, seed: int = 1234, keep_dense: bool = False) -> Workload:
    """Build q and the packed tiers of ``cfg`` on ``device`` from seeded host data."""
    gen = torch.Generator().manual_seed(seed)
    B, hkv, hd = cfg.batch, cfg.hkv, cfg.hd
    q = torch.randn(B, cfg.hq, hd, generator=gen, dtype=torch.float32).to(torch.float16)
    if cfg.ragged_min:
        lens = torch.randint(cfg.ragged_min, cfg.prompt + 1, (B,), generator=gen).tolist()
    else:
        lens = [cfg.prompt] * B
    pk = _dense(gen, (B, hkv, cfg.prompt, hd), cfg.k_kind, seed + 1)
    pv = _dense(gen, (B, hkv, cfg.prompt, hd), "normal", seed + 2)
    dev_k = pk.to(device)
    dev_v = pv.to(device)
    if cfg.ragged_min:
        # each row is quantized on its own valid length and padded into the tier buffer
        seg = pack_kv(dev_k, dev_v, cfg.prompt_bits, GROUP)
        for b, L in enumerate(lens):
            if L == cfg.prompt:
                continue
            row = pack_kv(dev_k[b:b + 1, :, :L].contiguous(), dev_v[b:b + 1, :, :L].contiguous(),
                          cfg.prompt_bits, GROUP)
            for full, part in ((seg.key, row.key), (seg.value, row.value)):
                if full.axis == 2:    # K: [B, Hkv, hd, bytes] / [B, Hkv, hd, groups]
                    full.packed[b, :, :, :part.packed.shape[-1]] = part.packed[0]
                    full.packed[b, :, :, part.packed.shape[-1]:] = 0
                    full.scale[b, :, :, :part.scale.shape[-1]] = part.scale[0]
                    full.mins[b, :, :, :part.mins.shape[-1]] = part.mins[0]
                else:                 # V: [B, Hkv, S, bytes] / [B, Hkv, S, groups]
                    full.packed[b, :, :L] = part.packed[0]
                    full.scale[b, :, :L] = part.scale[0]
                    full.mins[b, :, :L] = part.mins[0]
        prompt = seg
    else:
        prompt = pack_kv(dev_k, dev_v, cfg.prompt_bits, GROUP)
    cold = []
    ck = cv = None
    if cfg.cold:
        ck = _dense(gen, (B, hkv, cfg.cold, hd), cfg.k_kind, seed + 3)
        cv = _dense(gen, (B, hkv, cfg.cold, hd), "normal", seed + 4)
        cold.append(pack_kv(ck.to(device), cv.to(device), cfg.cold_bits, GROUP))
    hk = _dense(gen, (B, hkv, cfg.hot, hd), cfg.k_kind, seed + 5)
    hv = _dense(gen, (B, hkv, cfg.hot, hd), "normal", seed + 6)
    # hot window lives in a larger buffer, as in the cache (capacity = hot + 16)
    cap = cfg.hot + 16
    hot_k = torch.zeros(B, hkv, cap, hd, dtype=torch.float16, device=device)
    hot_v = torch.zeros(B, hkv, cap, hd, dtype=torch.float16, device=device)
    hot_k[:, :, :cfg.hot] = hk.to(device)
    hot_v[:, :, :cfg.hot] = hv.to(device)
    tiers = LayerTiers(prompt=prompt, cold=cold, hot_k=hot_k, hot_v=hot_v, hot_len=cfg.hot)
    plens = torch.tensor(lens, dtype=torch.int32, device=device) if cfg.ragged_min else None
    wl = Workload(cfg, q.to(device), tiers, plens, lens)
    if keep_dense:
        wl.dense_k = [pk, ck, hk]
        wl.dense_v = [pv, cv, hv]
    return wl


def tiers_algorithmic_bytes(tiers: LayerTiers, hq: int) -> int:
    """Algorithmic bytes of one decode step over ``tiers`` (every packed segment at its own
    length and width, the hot window, q and the output)."""
    B, hkv, _, hd = tiers.hot_k.shape
    total = 0
    for s in [tiers.prompt, *tiers.prompt_extensions, *tiers.cold]:
        total += _packed_bytes(s.key.orig_shape[2], hd, s.key.bits) * hkv * B
    return total + 4 * hd * tiers.hot_len * hkv * B + 2 * 2 * B * hq * hd


def make_long_generation(cfg: Config, generated: int, device, seed: int = 1234,
                         lazy_g: int = 16, keep_ratio: float = 1.0,
                         window: int = 32) -> Workload:
    """``cfg``'s batch-1 cache after ``generated`` decode tokens under lazy cooling: the
    prompt tier, ``cfg``'s cold tier, one cold segment of ``round(lazy_g * keep_ratio)``
    tokens at ``cfg.cold_bits`` per ``lazy_g`` generated tokens (packed as the cooling
    launch packs them) and a hot window of ``window`` + 8 tokens."""
    wl = make_workload(cfg, device, seed=seed)
    gen = torch.Generator().manual_seed(seed + 7)
    keep = max(1, round(lazy_g * keep_ratio))
    B, hkv, hd = cfg.batch, cfg.hkv, cfg.hd
    n_seg = max(0, generated - window) // lazy_g
    segs = []
    for _ in range(n_seg):
        k = _dense(gen, (B, hkv, keep, hd), cfg.k_kind, seed)
        v = _dense(gen, (B, hkv, keep, hd), "normal", seed)
        segs.append(pack_kv(k.to(device), v.to(device), cfg.cold_bits, GROUP))
    hot = window + 8
    hot_k = torch.zeros(B, hkv, window + lazy_g, hd, dtype=torch.float16, device=device)
    hot_v = torch.zeros_like(hot_k)
    hot_k[:, :, :hot] = _dense(gen, (B, hkv, hot, hd), cfg.k_kind, seed).to(device)
    hot_v[:, :, :hot] = _dense(gen, (B, hkv, hot, hd), "normal", seed).to(device)
    tiers = LayerTiers(prompt=wl.tiers.prompt, cold=list(wl.tiers.cold) + segs, hot_k=hot_k,
                       hot_v=hot_v, hot_len=hot)
    long_cfg = Config(f"{cfg.name}+{generated}gen", B, cfg.hq, hkv, hd, cfg.prompt,
                      cfg.prompt_bits, cfg.cold + n_seg * keep, cfg.cold_bits, hot, cfg.k_kind,
                      cfg.ragged_min)
    return Workload(long_cfg, wl.q, tiers, wl.prompt_lens, wl.prompt_lens_list)


def clone_tiers(t: LayerTiers) -> LayerTiers:
    """Deep copy of the device tensors (for buffer rotation in timing loops)."""
    def cseg(s: PackedKVSegment) -> PackedKVSegment:
        from dataclasses import replace
        return PackedKVSegment(
            replace(s.key, packed=s.key.packed.clone(), scale=s.key.scale.clone(),
                    mins=s.key.mins.clone()),
            replace(s.value, packed=s.value.packed.clone(), scale=s.value.scale.clone(),
                    mins=s.value.mins.clone()))
    return LayerTiers(prompt=cseg(t.prompt), prompt_extensions=[cseg(s) for s in t.prompt_extensions],
                      cold=[cseg(s) for s in t.cold], hot_k=t.hot_k.clone(), hot_v=t.hot_v.clone(),
                      hot_len=t.hot_len)
