"""Write tests/golden/jd_l0_11.npz from the reference's Jd.pt.

Jd.pt (src/molfm/models/e2former/Jd.pt) is a torch zip archive holding 12
float64 storages archive/data/{l} of shape (2l+1)^2.  They are read as raw
little-endian bytes; nothing in the archive is unpickled or executed.
"""
import sys
import zipfile
from pathlib import Path

import numpy as np

SRC = Path("/root/reference/src/molfm/models/e2former/Jd.pt")
OUT = Path(__file__).resolve().parent / "jd_l0_11.npz"

if __name__ == "__main__":
    src = Path(sys.argv[1]) if len(sys.argv) > 1 else SRC
    z = zipfile.ZipFile(src)
    arrs = {}
    for l in range(12):
        raw = z.read(f"archive/data/{l}")
        arrs[f"J{l}"] = np.frombuffer(raw, dtype="<f8").reshape(2 * l + 1, 2 * l + 1).copy()
    np.savez(OUT, **arrs)
    print(OUT, {k: v.shape for k, v in arrs.items()})
