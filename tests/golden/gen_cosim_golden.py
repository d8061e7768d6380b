"""Golden cosimulation tile dumps and PhaseB chain of the compiled reference
(build container only), for the synthetic C4 model and a one-token prompt,
run as `tmac_gguf c4.tmac --fpga-phaseb --dump-phaseb --dump-tiles 4
--dump-tiles-q5-0 3 --dump-tiles-q6-k 3` would (sim/tmac_gguf.cpp:2066-2177):
every --fpga flag on, the first position's matmuls recorded.

Stored in cosim.npz (no pickle):
  q8, q5, q6        the reference's three dump files, byte for byte
                    (cosim_tiles.bin, _q5_0.bin, _q6_k.bin: 16-byte header,
                    then 4992 / 6816 / 7616 bytes per tile)
  q5_fixed[3, 8]    the int64 results of the Q5_0 tiles and
  q6_fixed[3, 32]   of the Q6_K tiles as the tile primitives compute them for
                    the dumped inputs (the reference's dump overflows its
                    result array past the first tile and writes zeros there)
  phaseb_errors     phaseb_verify's error count
  bin_sha256, bin_size, hdr_sha256, hdr_size   /tmp/tb_phaseb.bin and .hdr
  hdr_head          the first 16 + 20 * ndesc bytes of the .hdr
  prompt, model_seed

    make -C oracle && python tests/golden/gen_cosim_golden.py
"""
from __future__ import annotations

import hashlib
import os
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tmac-zynq-fpga_amd"))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

from oracle import Q6_K, Reference  # noqa: E402
from tmq import model_synth, tmacfile  # noqa: E402
from gen_model_golden import MODEL_SEED, prompt_token  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))
NTILES = {"q8": 4, "q5": 3, "q6": 3}


def run(part, td):
    """one reference run in this process: "dumps" (the three tile dumps) or
    "phaseb" (the descriptor chain, verify, dump files).  The two run in
    separate processes: the reference's Q5_0 / Q6_K dumps overflow a stack
    array past their first tile, which corrupts the state of that run."""
    R = Reference()
    tok = prompt_token()
    path = os.path.join(td, "c4.tmac")
    R.model_load(path)
    R.model_set_flags(31)
    if part == "dumps":
        for which, k in enumerate(("q8", "q5", "q6")):
            assert R.lib.ref_dump_tiles_open(which, NTILES[k], os.path.join(td, f"{k}.bin").encode()) == 0
    else:
        assert R.lib.ref_phaseb_begin() == 0
    R.model_reset()
    hidden = np.zeros(R.HIDDEN, dtype=np.float32)
    R.model_step(hidden, tok, 0)                 # process_prompt([tok])
    R.model_logits_auto(hidden)                  # main's get_logits_q8
    R.lib.ref_phaseb_end()
    R.lib.ref_dump_tiles_close()
    if part == "phaseb":
        errors = R.lib.ref_phaseb_verify()
        R.lib.ref_phaseb_dump_files()                # /tmp/tb_phaseb.bin, .hdr
        np.save(os.path.join(td, "errors.npy"), np.int64(errors))


def main():
    import subprocess
    R = Reference()
    tok = prompt_token()
    with tempfile.TemporaryDirectory() as td:
        tmacfile.write(os.path.join(td, "c4.tmac"), model_synth.gen_model(MODEL_SEED))
        for part in ("dumps", "phaseb"):
            subprocess.check_call([sys.executable, os.path.abspath(__file__), "--part", part, td])
        dumps = {k: np.fromfile(os.path.join(td, f"{k}.bin"), dtype=np.uint8) for k in NTILES}
        errors = int(np.load(os.path.join(td, "errors.npy")))
    binb = open("/tmp/tb_phaseb.bin", "rb").read()
    hdrb = open("/tmp/tb_phaseb.hdr", "rb").read()
    os.remove("/tmp/tb_phaseb.bin")
    os.remove("/tmp/tb_phaseb.hdr")
    nd = int(np.frombuffer(hdrb[4:8], np.uint32)[0])
    # the fixed results: the tile primitives on the dumped inputs
    q5f = []
    for t in range(NTILES["q5"]):
        rec = dumps["q5"][16 + t * 6816: 16 + (t + 1) * 6816]
        res = np.zeros(8, np.int64)
        R.tile_q5_0_8x896(rec[:4928].copy(), rec[4928:6720].copy().view(np.int16),
                          rec[6720:6752].copy().view(np.float32), res, 0)
        q5f.append(res)
    q6f = []
    for t in range(NTILES["q6"]):
        rec = dumps["q6"][16 + t * 7616: 16 + (t + 1) * 7616]
        row0 = 32 * t  # tiles 0..2 of column group 0
        ri = np.zeros(896, np.float32)
        ri[row0:row0 + 32] = rec[7232:7360].copy().view(np.float32)
        res = np.zeros(896, np.int64)
        R.tile_kquant(Q6_K, rec[:6720].copy(), 32, rec[6720:7232].copy().view(np.int16), 256, ri, res, row0)
        q6f.append(res[row0:row0 + 32])
    np.savez_compressed(
        os.path.join(OUT, "cosim.npz"), model_seed=MODEL_SEED, prompt=np.array([tok], np.int32),
        q8=dumps["q8"], q5=dumps["q5"], q6=dumps["q6"], q5_fixed=np.array(q5f), q6_fixed=np.array(q6f),
        phaseb_errors=np.int64(errors), bin_sha256=hashlib.sha256(binb).hexdigest(), bin_size=np.int64(len(binb)),
        hdr_sha256=hashlib.sha256(hdrb).hexdigest(), hdr_size=np.int64(len(hdrb)),
        hdr_head=np.frombuffer(hdrb[:16 + 20 * nd], np.uint8))
    print(f"{nd} descriptors, {errors} verify errors, bin {len(binb)} B, hdr {len(hdrb)} B")


if __name__ == "__main__":
    if len(sys.argv) == 4 and sys.argv[1] == "--part":
        run(sys.argv[2], sys.argv[3])
    else:
        main()
