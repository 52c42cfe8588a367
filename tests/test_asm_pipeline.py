"""The decode kernel's two-tiles-ahead pipeline issues its K loads as inline asm, which the compiler does not
know to be in flight: on every path of the compiled gfx950 code, none of their destination registers may be
read, copied or reused before a wait that covers the load. Compiles paged_attention.hip (hipcc, no GPU) and
checks every decode instantiation that uses the pipeline."""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "nano-vllm-spec-decode_amd")
sys.path.insert(0, PKG)
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

from asm_paths import function_lines, unsafe_asm_loads  # noqa: E402

# attn_fwd<RT, kVarlen=false, kPaged=true, kWaves> with RT <= 2: the decode instantiations with the pipeline
DEEP = [f"_ZN2sd12_GLOBAL__N_18attn_fwdILi{rt}ELb0ELb1ELi{w}EEEvNS0_6ParamsE" for rt in (1, 2) for w in (8, 4, 2)]


@pytest.fixture(scope="module")
def device_asm(tmp_path_factory):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    import build_ext
    out = tmp_path_factory.mktemp("asm")
    cmd = [hipcc, *build_ext.DEVICE, *build_ext.COMMON, "--save-temps", "-c",
           os.path.join(build_ext.CSRC, "paged_attention.hip"), "-o", str(out / "pa.o")]
    res = subprocess.run(cmd, cwd=out, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-3000:]
    s = [f for f in os.listdir(out) if f.endswith(".s") and "gfx950" in f]
    assert s, os.listdir(out)
    return open(out / s[0]).read()


@pytest.mark.parametrize("symbol", DEEP)
def test_asm_k_loads_complete_before_use(device_asm, symbol):
    ins = function_lines(device_asm, symbol)
    bad, n = unsafe_asm_loads(ins)
    assert n >= 32, f"{symbol}: expected the pipeline's asm K loads, found {n}"
    assert not bad, bad[:4]


def test_checker_flags_a_register_touched_before_its_wait():
    load = ("global_load_dwordx4 v[4:7], v1, s[2:3]", True)
    bad, n = unsafe_asm_loads([load, ("v_mov_b32_e32 v5, 0", False), ("s_waitcnt vmcnt(0)", False)])
    assert n == 1 and bad
    assert not unsafe_asm_loads([load, ("s_waitcnt vmcnt(0)", False), ("v_mov_b32_e32 v5, 0", False)])[0]
    # vmcnt(1) with no later load leaves this one in flight
    bad, _ = unsafe_asm_loads([load, ("s_waitcnt vmcnt(1)", False),
                               ("v_mfma_f32_16x16x32_bf16 v[8:11], v[4:7], v[12:15], 0", False)])
    assert bad
    # ... but with one later load it covers this one
    bad, _ = unsafe_asm_loads([load, ("global_load_dwordx4 v[20:23], v1, s[2:3]", False), ("s_waitcnt vmcnt(1)", False),
                               ("v_mfma_f32_16x16x32_bf16 v[8:11], v[4:7], v[12:15], 0", False)])
    assert not bad
