"""The C ABI boundary: symbols, struct layouts and host-only entry points (no GPU)."""
import ctypes as C
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from voxgen_amd import abi, synth
from voxgen_amd.baselm import config_struct, kv_cache_bytes, rope_scaling_factor

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "voxhip.h"


def declared_functions() -> set:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(vx_[a-z0-9_]+)\s*\(", text))


def test_library_loads_and_exports_every_declared_symbol():
    lib = abi.load()
    names = declared_functions()
    assert len(names) > 60
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    assert set(abi.PROTOTYPES) == names, (set(abi.PROTOTYPES) ^ names)
    out = subprocess.run(["nm", "-D", "--defined-only", str(abi.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (vx_\w+)", out))
    assert names <= exported


def test_struct_layouts_match_the_c_compiler(tmp_path):
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "voxhip.h"', "int main(void){"]
    for cname, st in abi.STRUCT_SIZES.items():
        lines.append(f'printf("{cname} %zu\\n", sizeof({cname}));')
        for f, _ in st._fields_:
            lines.append(f'printf("{cname}.{f} %zu\\n", offsetof({cname}, {f}));')
    lines.append("return 0;}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    got = dict(l.split() for l in subprocess.run([str(exe)], capture_output=True, text=True,
                                                 check=True).stdout.splitlines())
    for cname, st in abi.STRUCT_SIZES.items():
        assert int(got[cname]) == C.sizeof(st), cname
        for f, _ in st._fields_:
            assert int(got[f"{cname}.{f}"]) == getattr(st, f).offset, (cname, f)


def test_push_structs_match_reference_field_order():
    # #[repr(C)] structs in src/baselm.rs:287-380, acoustic.rs:237-268: all 4-byte fields.
    assert [f for f, _ in abi.MatvecPush._fields_] == ["weight_offset", "rows", "cols", "dtype", "row_base", "alpha"]
    assert [f for f, _ in abi.QkvPush._fields_] == ["q_weight_offset", "k_weight_offset", "v_weight_offset",
                                                    "q_rows", "kv_rows", "cols", "q_dtype", "k_dtype",
                                                    "v_dtype", "row_base"]
    assert C.sizeof(abi.RopePush) == 28 and C.sizeof(abi.AttentionPush) == 24
    assert C.sizeof(abi.FusionPush) == 32 and C.sizeof(abi.LinearBiasPush) == 32


def test_top_k_reference_unit_test():
    # baselm.rs:1326-1329: top_k_logits([1,-2,5,3], 3) -> ids [2,3,0]
    lg = np.array([1.0, -2.0, 5.0, 3.0], np.float32)
    out = (abi.TopLogit * 3)()
    n = C.c_uint32()
    abi.call("vx_top_k_logits", lg.ctypes.data_as(C.POINTER(C.c_float)), 4, 3, out, C.byref(n))
    assert n.value == 3 and [out[i].token_id for i in range(3)] == [2, 3, 0]
    assert [out[i].logit for i in range(3)] == [5.0, 3.0, 1.0]


def test_top_k_skips_non_finite_and_clamps():
    lg = np.array([np.nan, 2.0, np.inf, -np.inf, 2.0, -1.0], np.float32)
    out = (abi.TopLogit * 8)()
    n = C.c_uint32()
    abi.call("vx_top_k_logits", lg.ctypes.data_as(C.POINTER(C.c_float)), 6, 8, out, C.byref(n))
    assert n.value == 3 and [out[i].token_id for i in range(3)] == [1, 4, 5]


def test_kv_cache_bytes_reference_unit_test():
    # baselm.rs:1332-1358: 28 layers x 32768 ctx x kv_dim 256 x f16 x (K+V)
    cfg = synth.baselm_config(context_length=32768, active_context=32768)
    assert kv_cache_bytes(cfg) == 939_524_096
    assert kv_cache_bytes(cfg) // 2 == 469_762_048


def test_rope_scaling_factor_host():
    cfg = synth.baselm_config(context_length=32768, original_context=4096)
    assert abs(rope_scaling_factor(cfg) - np.sqrt(1 + np.log(8) / np.log(4096))) < 1e-6
    assert rope_scaling_factor(synth.baselm_config()) == 1.0
    cfg["rope_longrope"] = 0
    assert rope_scaling_factor(cfg) == 1.0


def test_errors_are_codes_not_crashes():
    lib = abi.load()
    assert lib.vx_abi_version() == 2
    assert lib.vx_set_cancel_flag(None, None) == abi.STATUS_CODE["VX_ERR_INVALID_ARG"]
    st = lib.vx_alloc(None, 16, C.byref(abi.BUFP()))
    assert st == abi.STATUS_CODE["VX_ERR_INVALID_ARG"]
    assert b"null" in lib.vx_last_error()
    assert lib.vx_top_k_logits(None, 4, 1, None, None) == abi.STATUS_CODE["VX_ERR_INVALID_ARG"]
    with pytest.raises(abi.VxError) as e:
        abi.call("vx_sync", None)
    assert e.value.name == "VX_ERR_INVALID_ARG"


def test_product_package_has_no_oracle_dependency():
    """The shipped package never imports or loads the oracle."""
    for p in (ROOT / "voxgen_amd").rglob("*"):
        if p.suffix in (".py", ".cpp", ".hip", ".h", ".c"):
            text = p.read_text()
            assert "voxref" not in text and "liboracle" not in text, p
