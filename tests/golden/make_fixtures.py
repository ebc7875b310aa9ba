#!/usr/bin/env python3
"""Convert the reference's checked-in known-answer fixtures into compact npz files.

Reads (as data only) ``hw/test_data/{vecop,matmul,conv,pool,rowops}_test_data`` of the
reference checkout (default ``/root/reference``; Apache-2.0, copyright GradeBuilder SL and
Ivan Gubochkin) and writes ``tests/golden/<unit>.npz`` next to this script.  Each npz holds
the raw arrays of every case (``c<idx>_<name>``) plus ``manifest`` — the manifest rows as
a JSON string.  Only run in the build container; the GPU box never reads the reference.

Formats read (reference ``TestMatmulModel.cpp:161-190`` and siblings,
``kernels/rowops_rtl/scripts/gen_fixtures.py:1-22``):
  * vecop/matmul/conv/pool: one 16-bit hex value per line;
  * rowops: 16-byte words as 32 hex digits per line, byte 0 first; ``tables.hex`` the
    64 KiB table image; ``chains/`` the memory segment before / after each chain.
"""
import json
import os
import re
import sys

import numpy as np

REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
SRC = os.path.join(REF, "hw", "test_data")
OUT = os.path.dirname(os.path.abspath(__file__))


def read_hex16(path):
    with open(path) as f:
        vals = [int(line, 16) for line in f if line.strip()]
    return np.array(vals, dtype=np.uint16).view(np.int16)


def read_hex_words(path):
    out = bytearray()
    with open(path) as f:
        for line in f:
            line = line.strip()
            if line:
                out += bytes.fromhex(line)
    return np.frombuffer(bytes(out), dtype=np.uint8)


def manifest(path, ncols):
    rows = []
    with open(path) as f:
        for line in f:
            if line.startswith("#") or not line.strip():
                continue
            parts = line.split()
            nums = [int(p) for p in parts[:ncols]]
            label = " ".join(parts[ncols:])
            rows.append(nums + [label])
    return rows


def convert(unit, ncols, names, reader=read_hex16):
    d = os.path.join(SRC, f"{unit}_test_data")
    rows = manifest(os.path.join(d, "manifest.txt"), ncols)
    arrays = {}
    seen = set()
    uniq = []
    for r in rows:
        if r[0] in seen:        # a manifest may repeat its header block (conv)
            continue
        seen.add(r[0])
        uniq.append(r)
        for nm in names:
            p = os.path.join(d, f"test_{r[0]:02d}_{nm}.hex")
            if os.path.exists(p):
                arrays[f"c{r[0]}_{nm}"] = reader(p)
    arrays["manifest"] = np.array(json.dumps(uniq))
    np.savez_compressed(os.path.join(OUT, f"{unit}.npz"), **arrays)
    print(unit, len(uniq), "cases")


def convert_rowops():
    d = os.path.join(SRC, "rowops_test_data")
    rows = manifest(os.path.join(d, "manifest.txt"), 16)
    arrays = {}
    for r in rows:
        for nm in ("a", "b", "p", "c"):
            p = os.path.join(d, f"test_{r[0]:02d}_{nm}.hex")
            if os.path.exists(p):
                arrays[f"c{r[0]}_{nm}"] = read_hex_words(p)
    arrays["tables"] = read_hex_words(os.path.join(d, "tables.hex"))
    ch = os.path.join(d, "chains")
    jobs = manifest(os.path.join(ch, "manifest.txt"), 21)
    for cid in sorted({j[0] for j in jobs}):
        arrays[f"chain{cid}_mem"] = read_hex_words(os.path.join(ch, f"chain_{cid:02d}_mem.hex"))
        arrays[f"chain{cid}_out"] = read_hex_words(os.path.join(ch, f"chain_{cid:02d}_out.hex"))
    arrays["manifest"] = np.array(json.dumps(rows))
    arrays["chain_manifest"] = np.array(json.dumps(jobs))
    np.savez_compressed(os.path.join(OUT, "rowops.npz"), **arrays)
    print("rowops", len(rows), "cases,", len({j[0] for j in jobs}), "chains")


def convert_roms():
    """The VectorOP unit's ROM contents, parsed from the RTL's generated text tables
    (``kernels/vectorop_rtl/rtl/vo_act_rom.sv``: rom[BASE + t] = -round(256 f(-t/256)) per
    activation segment; ``vo_smx_rom.sv``: rom[k] = round(2^16 2^(-k/4096))) — the
    parsing of the reference's ``test_activations.py:96-110`` / ``test_softmax_unit.py:76-85``."""
    rtl = os.path.join(REF, "kernels", "vectorop_rtl", "rtl")
    text = open(os.path.join(rtl, "vo_act_rom.sv")).read()
    act = np.zeros(4096, np.int64)
    for a, v in re.findall(r"rom\[\s*(\d+)\] = 7'd(\d+)", text):
        act[int(a)] = int(v)
    seg = {name: (int(b), int(n)) for name, b, n in re.findall(
        r"(\w+)_BASE\s*=\s*12'd(\d+),\s*\w+_LEN\s*=\s*12'd(\d+);", text)}
    smx = np.zeros(4096, np.int64)
    for line in open(os.path.join(rtl, "vo_smx_rom.sv")):
        for part in line.split(";"):
            part = part.strip()
            if part.startswith("rom["):
                k, v = part[4:].split("] = 17'd")
                smx[int(k)] = int(v)
    np.savez_compressed(os.path.join(OUT, "roms.npz"), act_rom=act.astype(np.uint8),
                        act_segments=np.array(json.dumps(seg)), smx_tab=smx.astype(np.int32))
    print("roms", seg)


if __name__ == "__main__":
    convert_roms()
    convert("vecop", 11, ("a", "b", "c"))
    convert("matmul", 9, ("a", "b", "c"))
    convert("conv", 21, ("x", "w", "b", "y"))
    convert("pool", 18, ("x", "y"))
    convert_rowops()
