"""The C ABI library (no GPU needed): it loads, exports every function include/*.h declares, reports its
version/arch/error texts, sizes its scratch, and rejects bad arguments before enqueueing anything.

Every call below that passes placeholder pointers is constructed to fail argument validation, which runs before any
HIP call; no kernel is launched.
"""

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from ebr_amd import _capi

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))


def _declared():
    names = set()
    for h in HEADERS:
        names |= set(re.findall(r"^\s*(?:const\s+char\s*\*|int64_t|int)\s+(ebr_\w+)\s*\(", h.read_text(), re.M))
    return sorted(names)


def test_header_declares_the_expected_entry_points():
    assert _declared() == sorted(_capi.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _capi.load()
    for name in _declared():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(_capi.LIB_PATH)], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\b(ebr_(?:attn|rope|descent|block)_\w+)\b", out))
    assert exported == set(_declared())


def test_version_arch_and_error_texts():
    lib = _capi.load()
    assert lib.ebr_attn_abi_version() == _capi.ABI_VERSION == 3
    assert lib.ebr_attn_arch() == b"gfx950"
    for code in (0, 1, 2, 3, 4, 5, 6, 7):
        assert lib.ebr_attn_error_string(code)
    assert b"no-allocation" in lib.ebr_attn_error_string(_capi.ERR_NOALLOC_SIZE)
    assert b"unknown" in lib.ebr_attn_error_string(77)
    assert lib.ebr_attn_error_string(_capi.ERR_HIP_BASE + 1)  # hipErrorInvalidValue text


def test_scratch_sizes():
    lib = _capi.load()
    assert lib.ebr_attn_scratch_bytes(_capi.OP_FWD, 64, 8, 900, 64) == 0
    assert lib.ebr_attn_scratch_bytes(_capi.OP_BWD, 768, 8, 81, 64) == 0  # one-workgroup shapes need none
    assert lib.ebr_attn_scratch_bytes(_capi.OP_BWD_BWD, 768, 8, 128, 64) == 0
    assert lib.ebr_attn_scratch_bytes(_capi.OP_BWD, 64, 8, 900, 64) == 64 * 8 * 900 * 4
    assert lib.ebr_attn_scratch_bytes(_capi.OP_BWD_BWD, 64, 8, 900, 64) == 3 * 64 * 8 * 900 * 4
    # head dims above 128 run the two streamed launches at every L, so short sequences need the statistics too
    assert lib.ebr_attn_scratch_bytes(_capi.OP_BWD, 2, 4, 40, 256) == 2 * 4 * 40 * 4
    assert lib.ebr_attn_scratch_bytes(_capi.OP_BWD_BWD, 2, 4, 40, 136) == 3 * 2 * 4 * 40 * 4


def _str(*s):
    return (ctypes.c_int64 * 3)(*s)


P = 0x100000  # 16-byte aligned placeholder address; validation fails before it could be used
MIS = P + 8  # misaligned


def _fwd(dtype=1, B=1, H=1, L=4, D=64, q=P, qs=(0, 0, 64), o=P, lse=P):
    lib = _capi.load()
    s = _str(*qs)
    return lib.ebr_attn_fwd(dtype, B, H, L, D, ctypes.c_float(0.125), q, s, P, s, P, s, o, lse, None)


@pytest.mark.parametrize(
    "kwargs,code",
    [
        (dict(dtype=4), 1),  # unknown dtype
        (dict(dtype=-1), 1),
        (dict(dtype=3, D=257), 2),  # fp64: any D up to 256
        (dict(dtype=3, q=P + 4), 3),  # fp64 rows need 8-byte alignment
        (dict(D=264), 2),  # D > 256
        (dict(dtype=0, D=260), 2),  # fp32: D > 256
        (dict(D=60), 2),  # not a multiple of 8 for bf16
        (dict(dtype=0, D=62), 2),  # not a multiple of 4 for fp32
        (dict(L=0), 2),
        (dict(B=0), 2),
        (dict(q=0), 4),  # NULL input
        (dict(o=0), 4),  # NULL output
        (dict(q=MIS), 3),  # misaligned base
        (dict(qs=(0, 0, 60)), 3),  # row stride of 120 bytes
    ],
)
def test_fwd_rejects_bad_arguments(kwargs, code):
    assert _fwd(**kwargs) == code


def test_bwd_and_bwd_bwd_reject_bad_arguments():
    lib = _capi.load()
    s = _str(0, 0, 64)
    # dtype check comes first
    rc = lib.ebr_attn_bwd(7, 1, 1, 4, 64, ctypes.c_float(0.125), P, s, P, s, P, s, P, P, P, s, P, P, P, None, None)
    assert rc == 1
    # NULL dq
    rc = lib.ebr_attn_bwd(1, 1, 1, 4, 64, ctypes.c_float(0.125), P, s, P, s, P, s, P, P, P, s, 0, P, P, None, None)
    assert rc == 4
    # long L needs scratch: NULL scratch is rejected (this check follows the pointer checks)
    rc = lib.ebr_attn_bwd_bwd(
        1, 1, 1, 200, 64, ctypes.c_float(0.125),
        P, s, P, s, P, s, P, P, P, s, P, s, P, s, P, s, P, P, P, P, None, None,
    )  # fmt: skip
    assert rc == 5
    # negative stride
    rc = lib.ebr_attn_bwd_bwd(
        1, 1, 1, 4, 64, ctypes.c_float(0.125),
        P, _str(0, 0, -64), P, s, P, s, P, P, P, s, P, s, P, s, P, s, P, P, P, P, None, None,
    )  # fmt: skip
    assert rc == 3


def test_check_maps_codes_to_reference_exceptions():
    with pytest.raises(TypeError):
        _capi.check(1, "x")
    with pytest.raises(ValueError):
        _capi.check(2, "x")
    with pytest.raises(RuntimeError):
        _capi.check(3, "x")
    with pytest.raises(ValueError, match="plan"):
        _capi.check(_capi.ERR_PLAN, "x")
    with pytest.raises(RuntimeError, match="hip|error|invalid"):
        _capi.check(_capi.ERR_HIP_BASE + 1, "x")
    _capi.check(0, "x")


def test_build_recipe_targets_gfx950_without_packed_fp32():
    from ebr_amd import build

    flags = build.compile_flags()
    assert "--offload-arch=gfx950" in flags
    i = flags.index("-packed-fp32-ops")
    assert flags[i - 1] == "-Xclang" and flags[i - 2] == "-target-feature"


def test_build_forwards_extra_flags_to_compile_and_link(monkeypatch, tmp_path):
    """build() passes its extra flags to every compile and (bar -I / -D / -U) to the link, with one target arch."""
    from ebr_amd import build

    cmds = []

    def fake_run(cmd, verbose):
        cmds.append(cmd)
        Path(cmd[-1]).write_bytes(b"")
        return ""

    monkeypatch.setattr(build, "_run", fake_run)
    monkeypatch.setattr(build, "hipcc", lambda: "hipcc")
    monkeypatch.setattr(build, "OUT_DIR", tmp_path)
    extra = ("-fgpu-rdc", "-DEBR_PROBE=1", "-g", "-I/tmp/x")
    out = build.build(extra_flags=extra, jobs=1, arch="gfx950")
    assert out == tmp_path / build.LIB_NAME
    compiles = [c for c in cmds if "-c" in c]
    (link,) = [c for c in cmds if "-shared" in c]
    assert len(compiles) == len(build.SOURCES)
    for c in compiles:
        assert all(f in c for f in extra) and "--offload-arch=gfx950" in c
    assert "-fgpu-rdc" in link and "-g" in link and "--offload-arch=gfx950" in link
    assert not any(f.startswith(("-D", "-I")) for f in link)


def test_noalloc_entry_rejects_shapes_beyond_its_array_before_any_hip_call():
    """ebr_attn_bwd_bwd_noalloc checks the row-statistics size against EBR_NOALLOC_SCRATCH_BYTES first (no GPU needed:
    nothing is looked up or enqueued), and otherwise validates arguments exactly as ebr_attn_bwd_bwd does."""
    lib = _capi.load()
    z = (ctypes.c_int64 * 3)(0, 0, 0)
    tail = [16, z] * 3 + [16, 16] + [16, z] * 4 + [16, 16, 16, 16, None]
    B, H, L, D = 600, 8, 900, 64
    assert lib.ebr_attn_scratch_bytes(_capi.OP_BWD_BWD, B, H, L, D) > _capi.NOALLOC_SCRATCH_BYTES
    assert lib.ebr_attn_bwd_bwd_noalloc(_capi.DTYPE_BF16, B, H, L, D, ctypes.c_float(0.125), *tail) == 6
    assert lib.ebr_attn_bwd_bwd_noalloc(_capi.DTYPE_BF16, 0, H, L, D, ctypes.c_float(0.125), *tail) == 2  # B < 1
    assert lib.ebr_attn_bwd_bwd_noalloc(_capi.DTYPE_BF16, 2, 2, 81, 64, ctypes.c_float(0.125), *tail[:-5],
                                        None, 16, 16, 16, None) == 4  # hq NULL: L <= 128 needs no scratch lookup


def test_plan_entries_reject_unknown_plans_and_fp64_plans_before_any_hip_call():
    """The *_plan entry points check the plan (a family code, EBR_PLAN_AUTO only for fp64) with the other arguments,
    before anything is enqueued; placeholder pointers never reach a kernel."""
    lib = _capi.load()
    s = (ctypes.c_int64 * 3)(64 * 8, 64 * 8, 64)
    p = ctypes.c_void_p(16)  # aligned, never dereferenced
    for dtype, plan in ((_capi.DTYPE_BF16, 9), (_capi.DTYPE_BF16, -1), (_capi.DTYPE_F64, _capi.PLAN_GENERIC)):
        rc = lib.ebr_attn_fwd_plan(dtype, 1, 1, 8, 64, ctypes.c_float(0.125), p, s, p, s, p, s, p, p, None, plan)
        assert rc == _capi.ERR_PLAN, (dtype, plan, rc)


def test_integration_guide_stubs_compile_and_call_declared_entry_points():
    """The ctypes stubs the integration guide shows maintainers compile, and call only entry points the headers
    declare (their GPU test runs them against the oracle)."""
    import ast

    text = (ROOT / "INTEGRATION.md").read_text()
    stubs = [b for b in re.findall(r"```python\n(.*?)```", text, re.S) if "ctypes stub over libebr_attn.so" in b]
    assert len(stubs) == 3
    declared = set(_declared())
    for src in stubs:
        tree = ast.parse(src)
        called = {
            n.func.attr
            for n in ast.walk(tree)
            if isinstance(n, ast.Call) and isinstance(n.func, ast.Attribute)
            and isinstance(n.func.value, ast.Name) and n.func.value.id == "_lib"
        }
        assert called and called <= declared, called - declared
