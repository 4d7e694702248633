"""Convert the reference's golden vectors (test_data.zip) to tests/golden/test_data.npz.

The reference ships test_data.zip (written by flash_hog/_jax_refs/jax_impl.py:404-477
and :594-654): torch-saved fp32 tensors for one non-causal head, N_Q=128,
N_K=256, d=64, scale 1/8, inputs q,k,v,o,do,ddq,ddk,ddv,L and the outputs of
attn_bwd_bwd_stats, dq2,dk2,dv2,ddo. This script reads them with
torch.load(weights_only=True), which executes nothing from the file, and stores
the same arrays as float32 in an .npz fixture. Run it in the container that
holds the reference:

    python tests/golden/make_golden.py [path/to/test_data.zip]
"""

import io
import pathlib
import sys
import zipfile

import numpy as np
import torch

OUT = pathlib.Path(__file__).resolve().parent / "test_data.npz"
NAMES = ["q", "k", "v", "o", "do", "ddq", "ddk", "ddv", "L", "dq2", "dk2", "dv2", "ddo"]


def main(argv):
    src = pathlib.Path(argv[1] if len(argv) > 1 else "/root/reference/test_data.zip")
    arrays = {}
    with zipfile.ZipFile(src) as z:
        for entry in z.namelist():
            stem = pathlib.PurePosixPath(entry).stem
            if entry.endswith(".pt") and stem in NAMES:
                t = torch.load(io.BytesIO(z.read(entry)), weights_only=True)
                arrays[stem] = t.numpy().astype(np.float32)
    missing = set(NAMES) - set(arrays)
    if missing:
        raise SystemExit(f"missing tensors in {src}: {sorted(missing)}")
    np.savez_compressed(OUT, **arrays)
    print(OUT, {k: v.shape for k, v in arrays.items()})


if __name__ == "__main__":
    main(sys.argv)
