"""Writes hybrid_fixture_header.json: the config.json and the tensor names,
dtypes and shapes (no tensor bytes) of the reference's end-to-end fixture
tests/fixtures/hybrid/ (read as data: the JSON config and the safetensors
header).  Run in a container that holds the reference at /root/reference."""
import json
import os
import struct
import sys

SRC = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/tests/fixtures/hybrid"
here = os.path.dirname(os.path.abspath(__file__))
with open(os.path.join(SRC, "config.json")) as f:
    config = json.load(f)
with open(os.path.join(SRC, "model.safetensors"), "rb") as f:
    (n,) = struct.unpack("<Q", f.read(8))
    header = json.loads(f.read(n))
header.pop("__metadata__", None)
tensors = {k: {"dtype": v["dtype"], "shape": v["shape"]} for k, v in sorted(header.items())}
with open(os.path.join(here, "hybrid_fixture_header.json"), "w") as f:
    json.dump({"config": config, "tensors": tensors}, f, indent=0, sort_keys=True)
print(len(tensors), "tensors")
