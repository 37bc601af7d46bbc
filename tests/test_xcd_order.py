"""CPU test of the engine's XCD-ordered QKV row permutation (``Engine._qkv_xcd_order``).

For the M <= 2 GEMV the engine permutes the rows of each layer's QKV weight so that GEMV
workgroup g (which runs on XCD g mod 8) produces only rows of KV head group g mod 8: that
head's 4 query heads, its key and its value rows. The attention workgroup for that head runs
on the same XCD. Checked here on the Qwen3-4B shapes: the order is a permutation, every
workgroup's rows belong to one head group, and that group is g mod 8. Incompatible shapes
give None.
"""

import types

import torch

import engine as engine_mod
from qwen_hip import ops


def _stub(Nq, Nkv, D, H):
    spec = types.SimpleNamespace(Nq=Nq, Nkv=Nkv, D=D, H=H, qkv_width=(Nq + 2 * Nkv) * D)
    return types.SimpleNamespace(spec=spec, device=None)


def _group_of(row, Nq, Nkv, D):
    qd = Nq // Nkv * D
    if row < Nq * D:
        return row // qd
    if row < (Nq + Nkv) * D:
        return (row - Nq * D) // D
    return (row - (Nq + Nkv) * D) // D


def test_qwen4b_order_puts_each_head_group_on_one_xcd(monkeypatch):
    monkeypatch.setattr(ops, "gemv_config", lambda M, N, K, epi, device=None: (256, 8))
    Nq, Nkv, D, H = 32, 8, 128, 2560
    order = engine_mod.Engine._qkv_xcd_order(_stub(Nq, Nkv, D, H))
    N = (Nq + 2 * Nkv) * D
    assert order is not None and order.shape == (N,)
    assert torch.equal(torch.sort(order).values, torch.arange(N))
    rows = N // 256
    for g in range(256):
        groups = {_group_of(int(r), Nq, Nkv, D) for r in order[g * rows:(g + 1) * rows]}
        assert groups == {g % engine_mod.XCDS}, (g, groups)
    # within a head group the rows keep their natural order (q heads, then k, then v)
    for h in range(Nkv):
        mine = [int(order[p]) for p in range(N) if (p // rows) % 8 == h]
        assert mine == sorted(mine)


def test_incompatible_shapes_give_none(monkeypatch):
    monkeypatch.setattr(ops, "gemv_config", lambda M, N, K, epi, device=None: (256, 8))
    assert engine_mod.Engine._qkv_xcd_order(_stub(8, 2, 128, 512)) is None      # 2 KV heads
    monkeypatch.setattr(ops, "gemv_config", lambda M, N, K, epi, device=None: (304, 8))
    assert engine_mod.Engine._qkv_xcd_order(_stub(32, 8, 128, 2560)) is None    # 6144 rows over 304
