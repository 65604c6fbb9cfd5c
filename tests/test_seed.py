"""CPU: routing trace records and the seed builder (tools/make_seed.py restated in
a6000-custom-kernels_amd/seed.py; the record writer also in the C library).

Pinned by: a hand-counted trace; a trace built to reproduce the reference's own
seed fixture (tests/golden/moe_seed.txt, 144 tensors) line for line, with decode
counts in tie groups emitted lowest-count first (so the ranking must come from
the counts, ties from first-seen order) and prefill / single-expert records
mixed in that must not count; byte equality of the C writer's records with the
Python encoder."""
import io
import os
import struct
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
FIXTURE = ROOT / "tests" / "golden" / "moe_seed.txt"


@pytest.fixture(scope="module")
def seed(mc):
    import importlib
    return importlib.import_module("a6000_custom_kernels_amd.seed")


def test_record_layout(seed):
    rec = seed.encode_record("blk.3.ffn_up_exps.weight", [[5, 1], [7, 2]], 512)
    namelen, n_used, n_tok, n_exp = struct.unpack_from("<IIII", rec)
    assert (namelen, n_used, n_tok, n_exp) == (24, 2, 2, 512)
    assert rec[16:40] == b"blk.3.ffn_up_exps.weight"
    assert struct.unpack_from("<4i", rec, 40) == (5, 1, 7, 2)      # token-major
    assert len(rec) == 56
    long_name = "x" * 200
    assert struct.unpack_from("<I", seed.encode_record(long_name, [[1]], 4))[0] == 120


def test_hand_counted_trace(seed, tmp_path):
    A, B = "blk.0.ffn_up_exps.weight", "blk.0.ffn_down_exps.weight"
    buf = io.BytesIO()
    seed.append_record(buf, A, [[2, 7]], 8)
    seed.append_record(buf, B, [[1, 0]], 8)
    seed.append_record(buf, A, [[7, 5]], 8)
    seed.append_record(buf, A, [[7, 7], [7, 7]], 8)     # prefill record: read, not counted
    seed.append_record(buf, A, [[9, 2]], 8)             # 9 is out of range
    seed.append_record(buf, "ffn_gate_inp", [[1, 2]], 1)  # fewer than two experts: skipped
    seed.append_record(buf, A, [[5, 6]], 8)
    p = tmp_path / "t.bin"
    p.write_bytes(buf.getvalue())
    out = tmp_path / "s.txt"
    n_rec, counts = seed.make_seed(str(p), str(out))
    # A: 2 x2, 7 x2, 5 x2 (first seen in that order), 6 x1; B: 1, 0
    assert n_rec == 7
    assert out.read_text() == f"{A} 2,7,5,6\n{B} 1,0\n"
    assert counts[A] == {2: 2, 7: 2, 5: 2, 6: 1}


def test_truncated_record_is_an_error(seed):
    rec = seed.encode_record("t", [[1, 2, 3]], 8)
    with pytest.raises(ValueError):
        list(seed.read_trace(io.BytesIO(rec[:-2])))
    # a header cut short ends the trace quietly
    assert len(list(seed.read_trace(io.BytesIO(rec + rec[:10])))) == 1


def _fixture_trace(seed, lines):
    """A trace whose decode records rank every fixture line's ids exactly in the
    fixture's order: id k of n is picked 1 + (n - 1 - k) // 40 times, groups of
    equal count are emitted lowest count first, ids inside a group in fixture order."""
    buf = io.BytesIO()
    n_used = 8
    for name, ids in lines:
        n = len(ids)
        cnt = [1 + (n - 1 - k) // 40 for k in range(n)]
        order = []
        for c in sorted(set(cnt)):                       # first sightings, lowest counts first
            order += [ids[k] for k in range(n) if cnt[k] == c]
        for k in range(n):                               # remaining sightings
            order += [ids[k]] * (cnt[k] - 1)
        order += [-1] * (-len(order) % n_used)           # padding ids are out of range
        for r in range(0, len(order), n_used):
            seed.append_record(buf, name, [order[r:r + n_used]], 512)
            if r == 0:
                # a prefill record and a single-expert record that must not count
                seed.append_record(buf, name, [[ids[-1]] * n_used] * 4, 512)
                seed.append_record(buf, name + ".x", [[ids[-1]] * n_used], 1)
    return buf.getvalue()


def test_fixture_reproduced_line_for_line(seed, tmp_path):
    text = FIXTURE.read_text()
    lines = [(name, [int(t) for t in rest.split(",")])
             for name, _, rest in (ln.partition(" ") for ln in text.splitlines() if ln)]
    assert len(lines) == 144
    trace = tmp_path / "trace.bin"
    trace.write_bytes(_fixture_trace(seed, lines))
    out = tmp_path / "seed.txt"
    rc = seed.main([str(trace), str(out)])
    assert rc == 0
    assert out.read_text() == text
    assert seed.read_seed(str(out))["blk.47.ffn_gate_exps.weight"][:3] == [333, 183, 357]


def test_c_writer_matches_python_encoder(seed, mc, tmp_path):
    lib = mc.lib()
    p = tmp_path / "c_trace.bin"
    recs = [("blk.1.ffn_gate_exps.weight", np.array([[4, 9, 1]], dtype=np.int32), 64),
            ("blk.1.ffn_down_exps.weight", np.array([[3, 3], [8, 0]], dtype=np.int32), 64),
            ("n" * 150, np.array([[7]], dtype=np.int32), 16)]
    for name, ids, n_exp in recs:
        rc = lib.ggml_hip_moe_trace_append(str(p).encode(), name.encode(), ids.ctypes.data, ids.shape[1],
                                           ids.shape[0], n_exp)
        assert rc == 0, lib.ggml_hip_moe_last_error()
    assert lib.ggml_hip_moe_trace_close() == 0
    want = b"".join(seed.encode_record(name, ids, n_exp) for name, ids, n_exp in recs)
    assert p.read_bytes() == want
    # appends to an existing file, and refuses a record without ids
    ids = np.array([[1, 2]], dtype=np.int32)
    assert lib.ggml_hip_moe_trace_append(str(p).encode(), b"t", ids.ctypes.data, 2, 1, 4) == 0
    assert lib.ggml_hip_moe_trace_close() == 0
    assert p.read_bytes() == want + seed.encode_record("t", ids, 4)
    assert lib.ggml_hip_moe_trace_append(str(p).encode(), b"t", None, 2, 1, 4) != 0
    # no path and no GGML_HIP_MOE_TRACE / GGML_MOE_TRACE: nothing written, success
    if not (os.environ.get("GGML_HIP_MOE_TRACE") or os.environ.get("GGML_MOE_TRACE")):
        assert lib.ggml_hip_moe_trace_append(None, b"t", ids.ctypes.data, 2, 1, 4) == 0
