"""The Rust binding crate (crates/kernels-hip): its FFI declarations and
dispatch wrappers are generated from include/runit_hip.h and must match it
(no Rust toolchain exists in this image, so the crate itself is not compiled
here; this checks that it declares exactly the C ABI)."""
import os
import re
import subprocess
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CRATE = os.path.join(REPO, "crates", "kernels-hip")


def test_generated_files_are_current():
    r = subprocess.run([sys.executable, os.path.join(CRATE, "gen_bindings.py"), "--check"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr


def test_ffi_declares_every_header_function():
    from test_abi import header_functions
    ffi = open(os.path.join(CRATE, "src", "ffi.rs")).read()
    declared = set(re.findall(r"pub fn (rt_[a-z0-9_]+)\(", ffi))
    assert set(header_functions()) == declared


def test_dispatch_wraps_the_reference_names():
    src = open(os.path.join(CRATE, "src", "dispatch.rs")).read()
    for name in ("gemv_q8_0_f32in_f32out", "gemv_q8_0_add_f32_f32in", "fused_qkv_bias_q8_0_f32",
                 "fused_ffn_q8_0_f32", "fused_ffn_q4_0_f32", "gemv_q4k_f32in_f32out",
                 "rms_norm_f32_f32_f32g", "fused_rope_qk_f32", "kv_copy_to_cache_f32",
                 "decode_attention_f32", "argmax_f32", "add_f16_into_f32"):
        assert re.search(rf"pub fn {name}\(ctx: &HipContext", src), name
