"""The native C++ host layer (include/helix/helix.hpp) through its own test program
(tests/cpp/test_host.cpp, built by __graft_entry__.build()), plus an independent check of the
checkpoint bytes it writes.

The checkpoint body is bincode 1.x (the reference pins bincode = "1.3", training/Cargo.toml:30)
of Vec<CpuTensor> (backend-cpu/src/lib.rs:23-29, serde derive) with ndarray 0.15's array format
(features = ["serde"], backend-cpu/Cargo.toml:13). The expected bytes below are restated from
those published formats (little-endian fixed-width ints, u64 sequence lengths, u32 enum
variant indices, struct fields in order; ndarray = {v: u8 = 1, dim: [usize], data: [f32]});
the reference ships no checkpoint file to compare against and cannot be built here, so this
restatement is the pin."""
import struct
import subprocess
from pathlib import Path

import pytest

EXE = Path(__file__).resolve().parent / "cpp" / "helix_host_tests"


def run(args, timeout):
    if not EXE.exists():
        pytest.fail(f"{EXE} is not built (run __graft_entry__.build())")
    r = subprocess.run([str(EXE), *args], capture_output=True, text=True, timeout=timeout)
    print(r.stdout[-4000:], r.stderr[-2000:])
    return r


def expected_body(tensors):
    b = struct.pack("<Q", len(tensors))
    for shape, values in tensors:
        b += struct.pack("<B", 1)                                   # ndarray format version
        b += struct.pack("<Q", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
        b += struct.pack("<Q", len(values)) + b"".join(struct.pack("<f", v) for v in values)
        b += struct.pack("<Q", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
        b += struct.pack("<I", 9)                                   # DType::F32 (dtype.rs:8-37)
        b += struct.pack("<I", 0)                                   # Device::Cpu (device.rs:8-25)
    return b


def test_host_layer_cpu_cases_and_checkpoint_bytes(tmp_path):
    path = tmp_path / "ck.bin"
    r = run(["--cpu", str(path)], timeout=120)
    assert r.returncode == 0, "C++ host tests failed"
    raw = path.read_bytes()
    meta = b'{"epoch":3,"step":120}'
    assert raw[:4] == struct.pack(">I", len(meta))                  # tokio write_u32: big-endian
    assert raw[4:4 + len(meta)] == meta
    want = expected_body([((2, 3), [1, 2, 3, 4, 5, 6]), ((4,), [0.5, -0.5, 0.25, 8.0])])
    assert raw[4 + len(meta):] == want


@pytest.mark.gpu
def test_host_layer_gpu_cases():
    r = run(["--gpu"], timeout=300)
    assert r.returncode == 0, "C++ host tests failed on the GPU"
    assert "0 failed" in r.stdout
