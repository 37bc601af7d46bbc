"""CPU test of the engine's head-major QKV row permutation (``Engine._qkv_xcd_order``).

For the M <= 2 GEMV the engine permutes the rows of each layer's QKV weight so that block h
holds KV head group h (its 4 query heads, its key and its value rows), and runs the GEMV with 8
row groups: workgroup g (on XCD g mod 8) takes a share of block g mod 8. The attention
workgroup for that head runs on the same XCD. Checked here on the Qwen3-4B shapes: the order is
a permutation, and under the GEMV's group partition (``gemv_body``) every workgroup's rows
belong to head group g mod 8, for the 256-workgroup launch and the 248 projection workgroups
of the single-launch QKV + attention form. Incompatible shapes give None.
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


def _rows_of(g, G, N, groups=8):
    """Rows of workgroup g under the GEMV's group partition (csrc/gemv_impl.h, gemv_body)."""
    grp, j, Gg, Ng = g % groups, g // groups, G // groups, N // groups
    return range(Ng * grp + Ng * j // Gg, Ng * grp + Ng * (j + 1) // Gg)


def test_qwen4b_order_puts_each_head_group_on_one_xcd(monkeypatch):
    monkeypatch.setattr(ops, "gemv_config", lambda M, N, K, epi, device=None: (256, 8))
    Nq, Nkv, D, H = 32, 8, 128, 2560
    order = engine_mod.Engine._qkv_xcd_order(_stub(Nq, Nkv, D, H))
    N = (Nq + 2 * Nkv) * D
    assert order is not None and order.shape == (N,)
    assert torch.equal(torch.sort(order).values, torch.arange(N))
    for G in (256, 248, 240):
        covered = []
        for g in range(G):
            rows = _rows_of(g, G, N)
            groups = {_group_of(int(order[r]), Nq, Nkv, D) for r in rows}
            assert groups == {g % engine_mod.XCDS}, (G, g, groups)
            covered += list(rows)
        assert sorted(covered) == list(range(N))
    # within a head group the rows keep their natural order (q heads, then k, then v)
    grp = N // Nkv
    for h in range(Nkv):
        mine = [int(order[p]) for p in range(h * grp, (h + 1) * grp)]
        assert mine == sorted(mine)


def test_incompatible_shapes_give_none(monkeypatch):
    monkeypatch.setattr(ops, "gemv_config", lambda M, N, K, epi, device=None: (256, 8))
    assert engine_mod.Engine._qkv_xcd_order(_stub(8, 2, 128, 512)) is None      # 2 KV heads
    monkeypatch.setattr(ops, "gemv_config", lambda M, N, K, epi, device=None: (300, 8))
    assert engine_mod.Engine._qkv_xcd_order(_stub(32, 8, 128, 2560)) is None    # 300 workgroups: not 8 groups
