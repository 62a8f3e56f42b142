"""Copies the reference's end-to-end fixture tests/fixtures/hybrid/ (its
config.json, model.safetensors and oracle.json: data files the reference's
own parity check src/bin/hybrid-parity.rs reads) into tests/golden/hybrid/,
byte for byte.  Run in a container that holds the reference at
/root/reference."""
import hashlib
import os
import shutil
import sys

SRC = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/tests/fixtures/hybrid"
DST = os.path.join(os.path.dirname(os.path.abspath(__file__)), "hybrid")
os.makedirs(DST, exist_ok=True)
for name in ("config.json", "model.safetensors", "oracle.json"):
    shutil.copyfile(os.path.join(SRC, name), os.path.join(DST, name))
    with open(os.path.join(DST, name), "rb") as f:
        print(name, hashlib.sha256(f.read()).hexdigest())
