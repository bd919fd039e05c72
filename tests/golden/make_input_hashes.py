"""Write input_sha256.json: SHA-256 of the first 2^20 elements of every
synthetic benchmark tensor (the generator is counter-based, so a prefix pins
the stream).  Run: python tests/golden/make_input_hashes.py"""
import hashlib
import json
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "pytorch-rs_amd"))
from trs_backend.configs import CONFIGS, generate  # noqa: E402

PREFIX = 1 << 20


def main():
    out = {"prefix_elements": PREFIX, "hashes": {}}
    for cfg, spec in CONFIGS.items():
        for name, *_ in spec["tensors"]:
            arr = generate(cfg, name, PREFIX)
            out["hashes"][f"{cfg}.{name}"] = hashlib.sha256(arr.tobytes()).hexdigest()
    (Path(__file__).parent / "input_sha256.json").write_text(json.dumps(out, indent=1) + "\n")


if __name__ == "__main__":
    main()
