"""Synthetic SSPA decode workloads of the benchmark configurations (seeded, reproducible).

Each request: bf16 K/V ~ N(0, 1) with 4 key outlier channels scaled x8, full pages of
``page`` tokens whose value tier is drawn per page from a seeded categorical over
(BF16, INT4, INT2), a compact INT4-K arena, and a Recent-FP ring filled with the newest
``recent`` tokens by single-token appends (the reference fills the ring the same way: the
cache is built from the historical tokens, then generated tokens are appended).
Draw order per request: query, key, value, then the recent tokens' K/V rows.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .policy import PageClass, plan_from_pages

TIER_CLASS = (int(PageClass.FP_PAGE), int(PageClass.INT4_PAGE), int(PageClass.INT2_PAGE))


@dataclass(frozen=True)
class DecodeConfig:
    name: str
    hq: int
    hkv: int
    lengths: tuple[int, ...]          # total cached tokens per request (historical + recent)
    tier_probs: tuple[float, float, float]
    recent: int = 128
    page: int = 64
    superblock: int = 32
    group: int = 32
    variant: str = "int4k"     # "int4k" (v_fourq_k_int4_compact), "int2k" (v_fourq_k_int2_compact),
                               # "bf16k" (v_fourq_k_bf16) or "matched" (matched-FP)
    dtype: str = "bfloat16"    # model dtype of Q/K/V: "bfloat16" or "float16" (values drawn in bf16
                               # and converted, exactly, so both dtypes hold the same numbers)
    gen_values: str = "int2"   # generated_value_precision: flushed values INT2 (released) or INT4


CONFIGS = {
    0: DecodeConfig("qwen25omni3b_b1_4k_int4", 16, 2, (4096,), (0.0, 1.0, 0.0), recent=0),
    1: DecodeConfig("qwen25omni3b_b1_32k_mixed", 16, 2, (32768,), (0.2, 0.5, 0.3)),
    2: DecodeConfig("qwen25omni7b_b4_ragged_8k_64k", 28, 4, (8192, 16384, 32768, 65536), (0.15, 0.45, 0.4)),
    3: DecodeConfig("minicpmo45_b1_128k_int2", 32, 8, (131072,), (0.0, 0.0, 1.0), superblock=128, group=128),
}


@dataclass
class RequestData:
    query: torch.Tensor        # [1, Hq, 128] bf16
    key: torch.Tensor          # [Hkv, S_hist, 128] bf16
    value: torch.Tensor
    recent_k: torch.Tensor     # [recent, Hkv, 128] bf16 (append order)
    recent_v: torch.Tensor
    page_offsets: torch.Tensor
    page_lengths: torch.Tensor
    page_classes: torch.Tensor
    outliers: torch.Tensor


def make_request(cfg: DecodeConfig, total: int, seed: int, device) -> RequestData:
    """Draw one request of ``total`` cached tokens on ``device`` from ``seed``."""
    dev = torch.device(device)
    gen = torch.Generator(device=dev).manual_seed(seed)
    cpu = torch.Generator().manual_seed(seed)
    hist = total - cfg.recent
    if hist <= 0 or hist % cfg.page:
        raise ValueError("historical tokens must be a positive multiple of the page size")
    d = 128
    query = torch.randn(1, cfg.hq, d, generator=gen, device=dev).to(torch.bfloat16)
    key = torch.randn(cfg.hkv, hist, d, generator=gen, device=dev)
    outliers = torch.randperm(d, generator=cpu)[:4].to(dev)
    key[:, :, outliers] *= 8.0
    key = key.to(torch.bfloat16)
    value = torch.randn(cfg.hkv, hist, d, generator=gen, device=dev).to(torch.bfloat16)
    rk = torch.randn(cfg.recent, cfg.hkv, d, generator=gen, device=dev)
    rk[:, :, outliers] *= 8.0
    rk = rk.to(torch.bfloat16)
    rv = torch.randn(cfg.recent, cfg.hkv, d, generator=gen, device=dev).to(torch.bfloat16)
    pages = hist // cfg.page
    probs = torch.tensor(cfg.tier_probs, dtype=torch.float)
    tiers = torch.multinomial(probs, pages, replacement=True, generator=cpu)
    classes = torch.tensor(TIER_CLASS, dtype=torch.long)[tiers]
    offsets = torch.arange(pages, dtype=torch.long) * cfg.page
    lengths = torch.full((pages,), cfg.page, dtype=torch.long)
    if cfg.dtype == "float16":
        query, key, value, rk, rv = (t.to(torch.float16) for t in (query, key, value, rk, rv))
    elif cfg.dtype != "bfloat16":
        raise ValueError("DecodeConfig.dtype must be bfloat16 or float16")
    return RequestData(query, key, value, rk, rv, offsets, lengths, classes, outliers)


def build_request_cache(cfg: DecodeConfig, data: RequestData, *, append_capacity: int = 260):
    """Build the packed cache on the GPU and fill the Recent-FP ring with the recent tokens."""
    from .cache import build_three_precision_cache
    from .splitk import append_recent_fp_triton

    hist = int(data.key.shape[1])
    plan = plan_from_pages(data.page_offsets, data.page_lengths, data.page_classes, recent_fp_capacity=128,
                           device=data.key.device)
    cache = build_three_precision_cache(
        data.key, data.value, plan, page_size=cfg.page if cfg.page in (16, 32, 64) else 32,
        key_quantization_superblock=cfg.superblock, int2_group_size=cfg.group,
        compact_key_append_capacity=append_capacity, recent_flush_size=128,
        matched_fp=cfg.variant == "matched", generated_value_precision=cfg.gen_values,
        cache_variant={"bf16k": "v_fourq_k_bf16", "int2k": "v_fourq_k_int2_compact"}.get(
            cfg.variant, "v_fourq_k_int4_compact"))
    for i in range(int(data.recent_k.shape[0])):
        append_recent_fp_triton(cache, data.recent_k[i][:, None], data.recent_v[i][:, None],
                                global_token_index=hist + i, logical_position=hist + i)
    return cache


def algorithmic_bytes(caches, hq: int, *, fused_append: bool = False) -> int:
    """Compulsory HBM bytes of one decode call over ``caches`` (one per request).

    Per request and KV head: INT4-K codes (64 B/token) + K superblock scale/zero
    (3 B x 128 channels per superblock), INT2-K codes (32 B/token) + scale/offset (4 B x 128 per
    superblock), or BF16-K rows (256 B/token); BF16-V 256 B, INT4-V 64 + 4 B, INT2-V 32 + 3*128/G B,
    Recent K+V 512 B per active token; plus Q and O (bf16) and, with a fused append, the new
    K/V rows read and written.
    """
    total = 0
    for c in caches:
        hkv = int(c.recent_fp_pool.fp_k.shape[0])
        ck, cv = c.compact_key, c.compact_value
        if ck is not None and ck.bit_width == 4:
            hist = ck.active_length
            k_bytes = hist * 64 + -(-hist // ck.superblock_size) * 3 * 128
        elif ck is not None:  # INT2-K: 32 B codes per token, fp16 scale and offset per channel and block
            hist = ck.active_length
            k_bytes = hist * 32 + -(-hist // ck.superblock_size) * 4 * 128
        else:  # bf16 key rows (matched-FP and v_fourq_k_bf16 caches)
            k_bytes = c.bf16_key.active_length * 256
        v2_bytes = 0 if cv is None else cv.active_length * (32 + 3 * (128 // cv.group_size))
        per_head = (k_bytes + c.fp_pool.token_count * 256 + c.int4_pool.token_count * 68 + v2_bytes
                    + c.recent_fp_pool.active_length * 512)
        total += hkv * per_head + 2 * hq * 128 * 2
        if fused_append:
            total += 2 * hkv * 128 * 2 * 2
    return int(total)
