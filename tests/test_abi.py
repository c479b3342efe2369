"""The C ABI library on the CPU: it loads, exports every entry point that
include/nmoe_hip.h declares, and answers the calls that need no GPU."""
import ctypes
import subprocess

import nmoe_hip as nh


def test_library_exports_every_declared_symbol():
    declared = nh.header_symbols()
    assert len(declared) >= 20
    out = subprocess.run(["nm", "-D", "--defined-only", nh.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = [s for s in declared if s not in exported]
    assert not missing, missing
    lib = nh.lib()
    for s in declared:
        assert hasattr(lib, s)


def test_binding_covers_header():
    assert set(nh.header_symbols()) == set(nh._SIGS)


def test_expert_sizes_match_reference():
    # expert_io.m:90-99
    assert nh.lib().nmoe_hip_expert_size(4) == 1769472
    assert nh.lib().nmoe_hip_expert_size(2) == 983040
    assert nh.lib().nmoe_hip_expert_size(3) == 0


def test_null_context_is_rejected():
    lib = nh.lib()
    assert lib.nmoe_hip_synchronize(None) == nh.EINVAL
    assert lib.nmoe_hip_create(0, 0, ctypes.byref(ctypes.c_void_p())) == nh.EINVAL
    assert lib.nmoe_hip_set_option(None, nh.OPT_FUSED_DECODE, 1) == nh.EINVAL
