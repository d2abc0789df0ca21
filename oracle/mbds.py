"""mbds.py — numpy restatement of the reference's preprocessed-dataset file
(.mbds, Dataset.swift:26-86) and of its tile-8 bin layout (bin_index,
Shaders.swift:37-39).

TEST INFRASTRUCTURE ONLY.  The parity tests use it to write and read .mbds
files independently of the library; nothing in macboost_amd/ imports it.

File layout (little-endian; Dataset.swift:26-41):
    u32 magic 0x4D424453 ("SDBM" on disk), u32 version 1, u32 tile width 8,
    u64 rows, u32 cols, u32 numBins,
    u32 nCat, nCat x u32 categorical indices (ascending),
    u32 namesLen, namesLen bytes (JSONEncoder().encode([String]) or nothing),
    u64 nEdges, nEdges x f32 (cols * (numBins - 2)),
    u64 nLabels, nLabels x f32 (rows),
    u64 nBins, nBins x u8 (ceil(cols/8) * rows * 8, tile-8 layout).
"""
import struct

import numpy as np

MAGIC = 0x4D424453
VERSION = 1
TILE = 8


def swift_names_json(names) -> bytes:
    """[String] as Foundation's JSONEncoder writes it: compact, '/' escaped
    as '\\/', control characters escaped."""
    out = []
    for s in names:
        e = []
        for ch in s:
            o = ord(ch)
            if ch == '"':
                e.append('\\"')
            elif ch == "\\":
                e.append("\\\\")
            elif ch == "/":
                e.append("\\/")
            elif ch == "\n":
                e.append("\\n")
            elif ch == "\r":
                e.append("\\r")
            elif ch == "\t":
                e.append("\\t")
            elif ch == "\b":
                e.append("\\b")
            elif ch == "\f":
                e.append("\\f")
            elif o < 0x20:
                e.append("\\u%04x" % o)
            else:
                e.append(ch)
        out.append('"' + "".join(e) + '"')
    return ("[" + ",".join(out) + "]").encode("utf-8")


def tile8(bins_fm: np.ndarray) -> np.ndarray:
    """Feature-major bins [cols][rows] -> tile-8 layout [ceil(cols/8)][rows][8]:
    feature f of row i at (f >> 3) * rows * 8 + i * 8 + (f & 7)
    (bin_index, Shaders.swift:37-39); pad bytes are 0."""
    cols, rows = bins_fm.shape
    g = (cols + 7) // 8
    out = np.zeros((g * 8, rows), np.uint8)
    out[:cols] = bins_fm
    return np.ascontiguousarray(out.reshape(g, 8, rows).transpose(0, 2, 1))


def write(path, rows, cols, num_bins, categorical, feature_names, edges, labels, bins) -> bytes:
    """BinnedDataset.save (Dataset.swift:26-41); returns the bytes written."""
    d = bytearray()
    d += struct.pack("<IIIQII", MAGIC, VERSION, TILE, rows, cols, num_bins)
    cats = sorted(categorical)
    d += struct.pack("<I", len(cats))
    for c in cats:
        d += struct.pack("<I", c)
    names = swift_names_json(feature_names) if feature_names is not None else b""
    d += struct.pack("<I", len(names)) + names
    e = np.ascontiguousarray(edges, dtype="<f4").ravel()
    d += struct.pack("<Q", e.size) + e.tobytes()
    lab = np.ascontiguousarray(labels, dtype="<f4").ravel()
    d += struct.pack("<Q", lab.size) + lab.tobytes()
    b = np.ascontiguousarray(bins, dtype=np.uint8).ravel()
    d += struct.pack("<Q", b.size) + b.tobytes()
    with open(path, "wb") as f:
        f.write(d)
    return bytes(d)
