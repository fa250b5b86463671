"""The C ABI without a GPU: the library loads, exports every symbol the header
declares, the ctypes table matches the header, and argument validation fails
with error codes and messages before any device work."""

from __future__ import annotations

import ast
import os
import re
import subprocess
import sys

import pytest

from infrared_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "infrared_amd.h")


def _declared() -> dict[str, int]:
    """Function name -> parameter count, parsed from the header."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(ir_\w+)\s*\(([^;{]*?)\)\s*;", text):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_library_is_built_and_loads():
    assert os.path.exists(_lib.LIB_PATH), "run __graft_entry__.build() first"
    assert _lib.lib().ir_version().decode().startswith("infrared_amd")


def test_every_declared_symbol_is_exported_and_bound():
    decl = _declared()
    assert {"ir_kv_scatter", "ir_paged_decode", "ir_paged_attention_masked", "ir_gather_slots"} <= set(decl)
    lib = _lib.lib()
    for name, nparams in decl.items():
        assert hasattr(lib, name), f"{name} not exported"
        assert name in _lib.SIGNATURES, f"{name} missing from the ctypes table"
        assert len(_lib.SIGNATURES[name][1]) == nparams, f"{name}: ctypes arity != header"
    assert set(_lib.SIGNATURES) <= set(decl)


def test_validation_errors_report_codes_and_messages():
    lib = _lib.lib()
    # unknown dtype
    rc = lib.ir_kv_scatter(None, 0, 0, None, 0, 0, None, None, 0, 0, 0, None, 1, 1, 64, 99, None, None)
    assert rc == -1 and b"dtype" in lib.ir_last_error()
    # zero tokens is a successful no-op (no device work)
    rc = lib.ir_kv_scatter(None, 0, 0, None, 0, 0, None, None, 0, 0, 0, None, 0, 1, 64, 2, None, None)
    assert rc == 0 and lib.ir_last_error() == b""
    # unsupported head_dim
    rc = lib.ir_paged_decode(
        None, 0, 0, None, None, 0, 0, 1, 16, None, 0, 1, None, None, 0, 0, 1, 8, 2, 96, 1.0, 2, 0,
        None, 0, None, 0, None, None,
    )
    assert rc == -2 and b"head_dim" in lib.ir_last_error()
    # heads not a multiple of kv heads
    rc = lib.ir_paged_decode(
        None, 0, 0, None, None, 0, 0, 1, 16, None, 0, 1, None, None, 0, 0, 1, 7, 2, 128, 1.0, 2, 0,
        None, 0, None, 0, None, None,
    )
    assert rc == -1 and b"multiple" in lib.ir_last_error()
    # a plan for a shape the plan does not take
    rc = lib.ir_paged_decode_plan(None, 0, 16, None, 2000, 28, 4, 16, 100, 512, 128, 2, 0, None, 0, None, None)
    assert rc == -1 and b"plannable" in lib.ir_last_error()
    # null pointers with work to do
    rc = lib.ir_paged_attention_masked(
        None, 0, 0, 0, None, None, 0, 0, 10, None, 0, 0, None, 0, 0, 0, 2, None, 0, 0, 0, 1, 1, 4,
        4, 2, 128, 1.0, 2, None, None, None,
    )
    assert rc == -1 and b"null" in lib.ir_last_error()
    # the packed-form check: unknown mask dtype, empty frame (no-op), null pointers
    rc = lib.ir_varlen_form_scan(None, 8, 1, 99, 4, 8, None, 1, 16, 100,
                                 None, None, None, None, None, None, 0, None, 0, 0, None)
    assert rc == -1 and b"dtype" in lib.ir_last_error()
    rc = lib.ir_varlen_form_scan(None, 8, 1, 2, 0, 8, None, 1, 16, 100,
                                 None, None, None, None, None, None, 0, None, 0, 0, None)
    assert rc == 0 and lib.ir_last_error() == b""
    rc = lib.ir_varlen_form_scan(None, 8, 1, 2, 4, 8, None, 1, 16, 100,
                                 None, None, None, None, None, None, 0, None, 0, 0, None)
    assert rc == -1 and b"null" in lib.ir_last_error()
    rc = lib.ir_varlen_form_scan(None, 8, 1, 2, 4, 8, None, 1, 16, -1,
                                 None, None, None, None, None, None, 0, None, 0, 0, None)
    assert rc == -1 and b"bad sizes" in lib.ir_last_error()
    # a host record too small for 4 rows' chunk starts and prefixes (checked before any pointer is used)
    p = 256
    rc = lib.ir_varlen_form_scan(p, 8, 1, 2, 4, 8, p, 1, 16, 100, p, p, p, p, p, p, 64, p, 16, 0, None)
    assert rc == -1 and b"host_record holds 16 int32, needs 17" in lib.ir_last_error()
    # block tables narrower than their stride allows, and a table pass with no tables
    rc = lib.ir_varlen_form_tables(None, 1, None, None, None, 2, 16, None, 4, 8, None)
    assert rc == -1 and b"bad sizes" in lib.ir_last_error()
    rc = lib.ir_varlen_form_tables(None, 1, None, None, None, 2, 16, None, 8, 8, None)
    assert rc == -1 and b"null" in lib.ir_last_error()



def test_decode_workspace_and_partition_helpers():
    lib = _lib.lib()
    p = lib.ir_paged_decode_default_partition(64, 4, 256, 16)
    assert p % 16 == 0 and 256 <= p <= 8192
    # one partition covers everything -> no workspace
    assert lib.ir_paged_decode_workspace_size(8, 14, 2, 64, 32, 16, 512) == 0
    # 4096-token tables with 512-token partitions: 8 partitions of fp32 partials
    ws = lib.ir_paged_decode_workspace_size(64, 28, 4, 128, 256, 16, 512)
    rows = 64 * 28 * 8
    assert ws >= rows * 128 * 4 + rows * 2 * 4
    # counters: one per sequence x KV head x group of <= 16 query heads
    assert lib.ir_paged_decode_num_counters(64, 28, 4) == 64 * 4
    assert lib.ir_paged_decode_num_counters(8, 64, 2) == 8 * 2 * 2
    assert lib.ir_paged_decode_num_counters(8, 28, 3) == 0  # not a GQA shape


def test_decode_plan_helpers():
    """The plan is offered for 1..1024 sequences with block sizes that are
    multiples of 16, and its size covers one 8-byte fact per tile."""
    lib = _lib.lib()
    assert lib.ir_paged_decode_plan_bytes(0, 28, 4, 256, 16) == 0
    assert lib.ir_paged_decode_plan_bytes(1025, 28, 4, 256, 16) == 0
    assert lib.ir_paged_decode_plan_bytes(64, 28, 4, 256, 8) == 0
    n = lib.ir_paged_decode_plan_bytes(64, 28, 4, 256, 16)
    assert n >= 64 * 4 * 256 * 8  # tiles of the full table capacity, 8 bytes each
    assert lib.ir_paged_decode_plan_bytes(64, 28, 4, 256, 32) >= 64 * 4 * 512 * 8
    assert lib.ir_paged_decode_planned_workspace_bytes(64, 28, 4, 128) >= 256 * 16 * 128 * 4


def _plan_bytes(num_seqs, max_q, n_rep, h_kv, d, cus=256, xcds=1, cols=128):
    """The plan layout the header documents, restated: 4-wavefront workgroups of
    cols // n_rep query tokens (two resident per CU; 128 columns, 64 for an
    fp32 plan), one entry per workgroup -- (items + the piece capacity, one
    piece per KV head of every workgroup slot) x KV heads, 1.5x that rounded
    to the XCD count when the plan places work on XCDs -- the counters, and
    (max, sum) + D fp32 per partial row of `cols` columns; each region
    256-byte aligned."""
    a = lambda x: (x + 255) // 256 * 256  # noqa: E731
    tq = cols // n_rep
    nqb = -(-max_q // tq)
    slots = 2 * cus
    cap = -(-slots // h_kv)
    rows = cap * h_kv * cols
    wgs = (num_seqs * nqb + cap) * h_kv
    entries = xcds * -(-(wgs * 3 // 2) // xcds) if xcds > 1 else wgs
    return a(entries * 8) + a(cap * h_kv * 4) + a(rows * 8) + a(rows * d * 4)


def test_prefill_plan_helpers():
    """A prefill plan's size follows its documented layout (8 or 2 chunks of
    512 tokens at 28 / 4 heads: 29 blocks of 18 tokens each, two workgroups per
    CU), nothing is planned for empty or invalid shapes, and a
    short plan buffer or a null pointer is refused before any device work."""
    lib = _lib.lib()
    x = lib.ir_paged_prefill_plan_xcds()
    assert x >= 1
    # enough for either kind of plan: 16-bit (128 columns) or fp32 (64)
    for args in ((8, 512, 7, 4, 128), (2, 512, 7, 4, 64), (1, 4096, 1, 8, 128)):
        b, q_len, n_rep, h_kv, d = args
        want = max(_plan_bytes(*args, xcds=x), _plan_bytes(*args, xcds=x, cols=64))
        assert lib.ir_paged_prefill_plan_bytes(b, q_len, n_rep * h_kv, h_kv, d) == want, args
    # more than 64 query heads per KV head: no fp32 plan, the 16-bit size
    assert lib.ir_paged_prefill_plan_bytes(1, 64, 100, 1, 64) == _plan_bytes(1, 64, 100, 1, 64, xcds=x)
    assert lib.ir_paged_prefill_plan_bytes(0, 512, 28, 4, 128) == 0
    assert lib.ir_paged_prefill_plan_bytes(8, 512, 28, 3, 128) == 0
    assert lib.ir_paged_prefill_plan_bytes(8, 512, 28, 4, 96) == 0
    rc = lib.ir_paged_prefill_plan(None, None, None, 600, 8, 4096, 512, 600, 16, 28, 4, 128, 0, None, 7, None)
    assert rc == -1 and b"plan of" in lib.ir_last_error()
    rc = lib.ir_paged_prefill_plan(None, None, None, 600, 8, 4096, 512, 600, 16, 28, 4, 128, 0, 256, 1 << 30, None)
    assert rc == -1 and b"null" in lib.ir_last_error()


def test_no_product_module_imports_triton_or_the_oracle():
    pkg = os.path.join(ROOT, "infrared_amd")
    for name in os.listdir(pkg):
        if not name.endswith(".py"):
            continue
        tree = ast.parse(open(os.path.join(pkg, name)).read())
        for node in ast.walk(tree):
            mods = []
            if isinstance(node, ast.Import):
                mods = [a.name for a in node.names]
            elif isinstance(node, ast.ImportFrom) and node.module:
                mods = [node.module]
            for m in mods:
                assert not m.startswith("triton"), f"{name} imports {m}"
                assert not m.startswith("oracle"), f"{name} imports {m}"


def test_missing_library_fails_loudly(tmp_path):
    code = (
        "import infrared_amd._lib as L\n"
        f"L.LIB_PATH = {str(tmp_path / 'absent.so')!r}\n"
        "try:\n    L.lib()\nexcept RuntimeError as e:\n    print('RAISED', e)\n"
    )
    res = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, cwd=ROOT)
    assert "RAISED" in res.stdout and "no non-HIP fallback" in res.stdout


def test_pool_rejects_cpu_device():
    import torch

    from infrared_amd import PagedKVPool

    with pytest.raises(RuntimeError, match="ROCm device"):
        PagedKVPool(1, 4, 16, 2, 64, torch.float32, device="cpu")
