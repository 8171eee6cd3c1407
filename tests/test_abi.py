"""C-ABI surface checks that need no GPU.

* every function declared in include/runit_hip.h is exported by
  librunit_hip.so and has a ctypes signature in the Python mirror;
* every kernel the host library resolves at context creation is present in
  the gfx950 code object;
* without a GPU, context creation fails with NoDevice (KernelError::NoDevice,
  crates/kernels/src/error.rs:4-21) and the reason is readable from
  rt_global_last_error, as MetalContext::new reports a missing device
  (crates/kernels/src/context.rs:163-170).
"""
import ctypes
import os
import re

import pytest

from runit_mac_amd import dispatch as d

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "runit_hip.h")
RUNTIME = os.path.join(REPO, "runit_mac_amd", "csrc", "runtime.cpp")


def header_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    src = re.sub(r"//[^\n]*", "", src)
    names = set(re.findall(r"\b(rt_[a-z0-9_]+)\s*\(", src))
    assert len(names) > 60, names
    return sorted(names)


def runtime_kernel_names():
    src = open(RUNTIME).read()
    block = src[src.index("kKernelNames[] = {"):]
    block = block[:block.index("};")]
    return re.findall(r'"(k_[a-z0-9_]+)"', block)


@pytest.mark.parametrize("name", header_functions())
def test_library_exports_header_symbol(name):
    lib = ctypes.CDLL(d.LIB_PATH)
    assert hasattr(lib, name), f"{name} declared in runit_hip.h but not exported"


def test_python_mirror_binds_every_symbol():
    lib = d.load_library()
    missing = [n for n in header_functions() if getattr(lib, n).argtypes is None]
    assert not missing, missing


def test_code_object_holds_every_resolved_kernel():
    # every code object of the build (one per kernel unit) together
    blob = b"".join(open(os.path.join(d.HSACO_PATH, f), "rb").read()
                    for f in sorted(os.listdir(d.HSACO_PATH)) if f.endswith(".hsaco"))
    names = runtime_kernel_names()
    assert len(names) > 80
    missing = [n for n in names if (n.encode() + b"\0") not in blob]
    assert not missing, missing


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU driver is present")
def test_no_device_raises_no_device():
    with pytest.raises(d.NoDevice) as ei:
        d.HipContext()
    assert "device" in str(ei.value).lower()


def test_missing_code_object_is_library_load_or_no_device():
    # NoDevice is checked first (context.rs:163-170 creates the device before
    # loading the library); with a device present, a bad path is LibraryLoad.
    with pytest.raises((d.NoDevice, d.LibraryLoad)):
        d.HipContext(code_object="/nonexistent/runit_kernels.hsaco")
