"""Autotune config lists re-tuned for MI355X (reference: src/enceladus/configs.py:19-127).

Tiles are BLOCK ∈ {64, 128, 256} per the MI355X sweep; `num_warps` counts 64-lane waves.
"""

from __future__ import annotations

from enceladus_amd.runtime.autotuner import Config


def _dtype_name(dt) -> str:
    return getattr(dt, "long_name", None) or str(dt).removeprefix("tl.")


def matmul_configs(dtype="float16") -> list[Config]:
    name = _dtype_name(dtype)
    out = []
    for bm in (64, 128, 256):
        for bn in (64, 128, 256):
            for bk in (32, 64, 128):
                if bm * bn > 256 * 128:
                    continue
                if name == "float32" and bk > 32:
                    continue
                nw = 8 if bm * bn >= 256 * 128 else 4
                out.append(Config({"BM": bm, "BN": bn, "BK": bk}, num_warps=nw))
    return out


def attention_configs(dtype="float16", head_dim: int = 128) -> list[Config]:
    out = []
    for bm in (64, 128, 256):
        for bn in (32, 64, 128):
            if head_dim >= 128 and bn > 64 and bm > 128:
                continue
            nw = max(1, min(8, bm // 32))
            out.append(Config({"BLOCK_M": bm, "BLOCK_N": bn}, num_warps=nw,
                              dot_warps=(nw, 1)))
    return out
