"""The C-ABI library loads (no GPU needed) and exports every symbol include/qwen_hip.h declares."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qwen_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:int|long long)\s+(qwen_\w+)\s*\(", text, flags=re.M)


def test_header_declares_entry_points():
    names = declared_symbols()
    assert len(names) >= 13 and len(set(names)) == len(names)


def test_library_exports_every_declared_symbol():
    from qwen_hip import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libqwen_hip.so not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_python_binding_covers_header():
    from qwen_hip import _lib
    assert set(_lib.SIGNATURES) == set(declared_symbols())


def test_header_argument_counts_match_binding():
    from qwen_hip import _lib
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    for name, (_, args) in _lib.SIGNATURES.items():
        m = re.search(name + r"\s*\((.*?)\);", text, flags=re.S)
        assert m, name
        nargs = len([a for a in m.group(1).split(",") if a.strip()])
        assert nargs == len(args), f"{name}: header {nargs} args, binding {len(args)}"


def test_workspace_queries_run_without_gpu():
    from qwen_hip import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libqwen_hip.so not built")
    # one counter per row (padded to 256 B), then split partials (m, l, acc[128]) per (row, split, head)
    assert _lib.query("qwen_attn_workspace_bytes", 1, 1, 32, 8, 128, 4) == 1 * 8 * 4 * 4 * (2 + 128) * 4 + 256
    assert _lib.query("qwen_attn_workspace_bytes", 1, 1, 32, 8, 128, 1) == 0      # one split: no workspace
    assert _lib.query("qwen_attn_workspace_bytes", 0, 1, 32, 8, 128, 4) == 0
    # split-K: a fixed counter region, then units * ks * (MT * ntw) fragments of 1 KB
    units = 2560 // 16
    counters = 65536     # fixed region: GEMMs of any shape share one workspace
    assert _lib.query("qwen_linear_workspace_bytes", 1, 2560, 1, 4) == units * 4 * 1024 + counters
    assert _lib.query("qwen_linear_workspace_bytes", 32, 2560, 1, 4) == units * 4 * 2048 + counters
    assert _lib.query("qwen_linear_workspace_bytes", 8, 2560, 1, 1) == 0


def test_ops_refuse_cpu_tensors():
    """The product path has no CPU fallback: ops raise instead of computing on the host."""
    import torch
    from qwen_hip import ops
    x = torch.zeros(2, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError):
        ops.rms_norm(x, torch.ones(128, dtype=torch.bfloat16), 1e-6)


def test_engine_refuses_without_gpu(tmp_path):
    import torch
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    from __graft_entry__ import SMOKE_CFG, write_random_model
    from engine import Engine
    with pytest.raises(RuntimeError):
        Engine(write_random_model(str(tmp_path), SMOKE_CFG))
