#!/usr/bin/env python3
"""Routing traces and hot-expert seed files for the pointer-table cache.

Trace record (one per MUL_MAT_ID; patches/trace-hook/ggml-cpu.c:1-9, :1597-1617),
little endian:

    u32 namelen, u32 n_used, u32 n_tok, u32 n_exp, char name[namelen], i32 ids[n_used * n_tok]

`name` is the expert tensor's name cut to 120 bytes; ids are token-major (ggml's
ids layout, n_used per token).  The library writes the same records from C
(`ggml_hip_moe_trace_append`).

Seed file (tools/make_seed.py:22-55): one line per expert tensor, in the order
the tensors first appear in the trace, `"<name> id,id,..."`, listing every
expert the decode records (n_tok == 1 and n_exp >= 2) picked, by descending
pick count, equal counts in the order first seen.  The cache seeds a tensor's
pool slots from the head of its line (`GGML_HIP_MOE_CACHE_SEED`).

Usage (the reference tool's arguments):

    python a6000-custom-kernels_amd/seed.py [trace.bin] [seed.txt]
"""
from __future__ import annotations

import argparse
import struct
from dataclasses import dataclass
from typing import BinaryIO, Dict, Iterable, Iterator, List, Sequence, Tuple

import numpy as np

_HDR = struct.Struct("<IIII")
NAME_MAX = 120


@dataclass
class TraceRecord:
    name: str
    n_used: int
    n_tok: int
    n_exp: int
    ids: np.ndarray          # int32 [n_tok, n_used]


def encode_record(name: str, ids, n_exp: int) -> bytes:
    """One trace record for the routing `ids` ([n_tok, n_used] int32) of tensor `name`."""
    a = np.ascontiguousarray(np.asarray(ids, dtype=np.int32))
    if a.ndim == 1:
        a = a.reshape(1, -1)
    if a.ndim != 2:
        raise ValueError("ids must be [n_tok, n_used]")
    raw = name.encode("utf-8")[:NAME_MAX]
    n_tok, n_used = a.shape
    return _HDR.pack(len(raw), n_used, n_tok, n_exp) + raw + a.astype("<i4").tobytes()


def append_record(f: BinaryIO, name: str, ids, n_exp: int) -> None:
    f.write(encode_record(name, ids, n_exp))


def read_trace(f: BinaryIO) -> Iterator[TraceRecord]:
    """Records of a trace stream; a header shorter than 16 bytes ends it (as the
    reference tool stops), a record cut inside its name or ids is an error."""
    while True:
        hdr = f.read(_HDR.size)
        if len(hdr) < _HDR.size:
            return
        namelen, n_used, n_tok, n_exp = _HDR.unpack(hdr)
        raw = f.read(namelen)
        body = f.read(4 * n_used * n_tok)
        if len(raw) < namelen or len(body) < 4 * n_used * n_tok:
            raise ValueError("truncated trace record")
        ids = np.frombuffer(body, dtype="<i4").astype(np.int32).reshape(n_tok, n_used)
        yield TraceRecord(raw.decode("utf-8", "replace"), n_used, n_tok, n_exp, ids)


def decode_counts(records: Iterable[TraceRecord]) -> Tuple[int, Dict[str, Dict[int, int]]]:
    """(records read, per tensor name: expert -> decode pick count), both dicts in
    first-appearance order.  Records with n_tok != 1 (prefill) or n_exp < 2 are
    read and counted as records but add no picks; ids outside [0, n_exp) are skipped."""
    counts: Dict[str, Dict[int, int]] = {}
    n_rec = 0
    for r in records:
        n_rec += 1
        if r.n_tok != 1 or r.n_exp < 2:
            continue
        c = counts.setdefault(r.name, {})
        for e in r.ids.reshape(-1).tolist():
            if 0 <= e < r.n_exp:
                c[e] = c.get(e, 0) + 1
    return n_rec, counts


def ranked(c: Dict[int, int]) -> List[int]:
    """Experts by descending count; Python's sort is stable, so equal counts keep
    first-seen order (the order collections.Counter.most_common gives)."""
    return [e for e, _ in sorted(c.items(), key=lambda kv: kv[1], reverse=True)]


def seed_lines(counts: Dict[str, Dict[int, int]]) -> List[str]:
    return [name + " " + ",".join(str(e) for e in ranked(c)) for name, c in counts.items()]


def make_seed(trace_path: str, out_path: str) -> Tuple[int, Dict[str, Dict[int, int]]]:
    """Reads a trace, writes the seed file; returns (records, counts)."""
    with open(trace_path, "rb") as f:
        n_rec, counts = decode_counts(read_trace(f))
    with open(out_path, "w") as f:
        for line in seed_lines(counts):
            f.write(line + "\n")
    return n_rec, counts


def read_seed(path: str) -> Dict[str, List[int]]:
    """A seed file as {tensor name: [ids in seed order]}."""
    out: Dict[str, List[int]] = {}
    with open(path) as f:
        for line in f:
            line = line.rstrip("\n")
            if not line:
                continue
            name, _, rest = line.partition(" ")
            out[name] = [int(t) for t in rest.split(",") if t]
    return out


def main(argv: Sequence[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description="Build a hot-expert seed file from a MoE routing trace.")
    ap.add_argument("trace", nargs="?", default="moe_trace.bin", help="routing trace (GGML_HIP_MOE_TRACE records)")
    ap.add_argument("out", nargs="?", default="moe_seed.txt", help="seed file to write")
    args = ap.parse_args(argv)
    n_rec, counts = make_seed(args.trace, args.out)
    print(f"records={n_rec} tensors={len(counts)} -> {args.out}")
    for name in list(counts)[:3]:
        c = counts[name]
        print(name, "top10:", ranked(c)[:10], "distinct:", len(c))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
