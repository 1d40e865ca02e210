"""Writes the committed golden fixtures from the reference's own data files.

The reference ships six fp32 golden sets produced by PyTorch's
scaled_dot_product_attention (raw little-endian float32, C-contiguous
[B,H,L,D]; written by scripts/generate_pytorch_reference.py:49-56 with the
shapes and seeds of :87-94).  No reference code is run or imported here: the
.bin files are read as data.

Committed (small, so they travel to the GPU box):
  * tiny  (1,1,4,8)   -- BASELINE config 1 exactly -- verbatim;
  * small (1,2,8,16)  -- verbatim;
  * hdim512 head 0    -- (1,1,64,512) slice of the (1,4,64,512) set.
The manifest records the sha256 of every original file so a test in this
container can re-check the full sets (hdim2048 is BASELINE config 2 exactly)
when /root/reference is present.

Usage: python tests/golden/make_fixtures.py [/root/reference]
"""
import hashlib
import json
import os
import sys

import numpy as np

SETS = [  # name, shape, seed  (scripts/generate_pytorch_reference.py:87-94)
    ("tiny", (1, 1, 4, 8), 42),
    ("small", (1, 2, 8, 16), 43),
    ("hdim512", (1, 4, 64, 512), 44),
    ("hdim2048", (1, 4, 64, 2048), 45),
    ("hdim4096", (1, 2, 32, 4096), 46),
    ("hdim8192", (1, 1, 16, 8192), 47),
]
VERBATIM = {"tiny", "small"}
HEAD_SLICE = {"hdim512": 0}


def main(ref_root: str) -> None:
    here = os.path.dirname(os.path.abspath(__file__))
    data_dir = os.path.join(ref_root, "pytorch_reference_data")
    manifest = {"source": "pytorch_reference_data/pytorch_ref_<name>_<T>.bin",
                "format": "float32 little-endian, C-contiguous [B,H,L,D]", "sets": {}}
    for name, shape, seed in SETS:
        entry = {"shape": list(shape), "seed": seed, "sha256": {}, "fixture": None}
        arrays = {}
        for t in ("Q", "K", "V", "output"):
            path = os.path.join(data_dir, f"pytorch_ref_{name}_{t}.bin")
            raw = open(path, "rb").read()
            entry["sha256"][t] = hashlib.sha256(raw).hexdigest()
            arrays[t] = np.frombuffer(raw, dtype="<f4").reshape(shape)
        if name in VERBATIM:
            for t, a in arrays.items():
                a.astype("<f4").tofile(os.path.join(here, f"{name}_{t}.bin"))
            entry["fixture"] = {"file": f"{name}_<T>.bin", "shape": list(shape)}
        elif name in HEAD_SLICE:
            h = HEAD_SLICE[name]
            fshape = (1, 1, shape[2], shape[3])
            for t, a in arrays.items():
                np.ascontiguousarray(a[:, h:h + 1]).astype("<f4").tofile(
                    os.path.join(here, f"{name}_h{h}_{t}.bin"))
            entry["fixture"] = {"file": f"{name}_h{h}_<T>.bin", "shape": list(fshape),
                                "slice": f"head {h}"}
        manifest["sets"][name] = entry
    with open(os.path.join(here, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
