"""python -m model <config>: the L2 traffic model of c3 (or another synthetic configuration) at
F = 128 and 256 under the three policies, printed as one JSON object."""
import json
import pathlib
import sys
import time

sys.path.insert(0, str(pathlib.Path(__file__).resolve().parents[1]))

import tcc_spmm_amd as T  # noqa: E402
import model  # noqa: E402

cfg = sys.argv[1] if len(sys.argv) > 1 else "c3"
csr = T.synth_csr(cfg)
fmt = T.convert_csr_to_sw32(csr.rows, csr.cols, csr)
out = {"config": cfg}
for feats in (128, 256):
    for pol in ("cold", "lru", "opt"):
        t = time.time()
        r = model.traffic(fmt, feats, pol)
        r["seconds"] = round(time.time() - t, 1)
        out[f"f{feats}_{pol}"] = r
        print(f"F{feats} {pol}: {r['bytes'] / 1e9:.2f} GB ({r['seconds']} s)", file=sys.stderr, flush=True)
print(json.dumps(out, indent=1))
