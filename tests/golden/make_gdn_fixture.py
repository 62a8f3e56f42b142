"""Extracts the GatedDeltaNet subset of the reference's held fixture
tests/fixtures/native-kernels.safetensors (used by the reference's
tests/native_kernels.rs:18-32, 64-79: one decode step at B=1, T=1, Hk=16,
Hv=48, d=128, non-zero initial state) into a small .npz golden file.

Only value heads 0..5 and the key heads they read (0..1, Hv/Hk = 3) are
kept: heads are independent, so the subset is an exact test.  The
safetensors file is parsed directly (8-byte header length, JSON header,
raw little-endian tensor bytes): a pure data read, since numpy has no bf16
dtype for the library loader to return.

    python tests/golden/make_gdn_fixture.py /root/reference/tests/fixtures/native-kernels.safetensors
"""
import os
import sys

import json
import struct

import numpy as np

HV_KEEP = 6
HK_KEEP = 2


_DTYPES = {"BF16": np.uint16, "F32": np.float32, "I32": np.int32, "U32": np.uint32}


def read_safetensors(path: str) -> dict:
    with open(path, "rb") as f:
        (n,) = struct.unpack("<Q", f.read(8))
        header = json.loads(f.read(n))
        base = 8 + n
        out = {}
        for name, meta in header.items():
            if name == "__metadata__" or meta["dtype"] not in _DTYPES:
                continue
            a, b = meta["data_offsets"]
            f.seek(base + a)
            buf = f.read(b - a)
            out[name] = np.frombuffer(buf, _DTYPES[meta["dtype"]]).reshape(meta["shape"]).copy()
    return out


def main(src: str) -> None:
    t = read_safetensors(src)
    out = {
        "q": t["q"][:, :, :HK_KEEP, :].copy(),       # bf16 bits [1,1,2,128]
        "k": t["k"][:, :, :HK_KEEP, :].copy(),
        "v": t["v"][:, :, :HV_KEEP, :].copy(),       # bf16 bits [1,1,6,128]
        "beta": t["beta"][:, :, :HV_KEEP].copy(),    # bf16 bits [1,1,6]
        "y": t["y"][:, :, :HV_KEEP, :].copy(),       # bf16 bits [1,1,6,128]
        "g": t["g"][:, :, :HV_KEEP].copy(),          # f32 [1,1,6]
        "initial": t["initial"][:, :HV_KEEP].copy(),  # f32 [1,6,128,128] (MLX [B,Hv,Dv,Dk])
        "state": t["state"][:, :HV_KEEP].copy(),
    }
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gdn_native_kernels_subset.npz")
    np.savez(dst, **out)
    print(dst, {k: (v.dtype, v.shape) for k, v in out.items()})


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else
         "/root/reference/tests/fixtures/native-kernels.safetensors")
