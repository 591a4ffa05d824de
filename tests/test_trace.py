"""FMT1 selection traces (CPU).  No trace ships with the reference, so the
fixtures are written here in the capture tool's layout
(tools/capture_miss_trace.py:316-317 header, :366-370 records); the reader is
pinned by hand-computed renamings, by the numpy restatement in the oracle
and by the error cases the reference's loader refuses
(src/workloads/miss_trace.cuh:81-131)."""
import struct

import numpy as np
import pytest

import ferry_amd as F
from oracle import pyoracle as O


def write_fmt1(path, records, R, S, L, page_tokens=16, block_tokens=4, kv=4, d=128, sel_pages=2,
               version=1, magic=b"FMT1"):
    """records[r][s][l] = list of u32 block ids, written as the capture tool does."""
    with open(path, "wb") as f:
        f.write(struct.pack("<4sIIIIIIIII", magic, version, R, S, L, page_tokens, block_tokens,
                            kv, d, sel_pages))
        for r in range(R):
            for s in range(S):
                for l in range(L):
                    blks = records[r][s][l]
                    f.write(struct.pack("<H", len(blks)))
                    if len(blks):
                        f.write(np.asarray(blks, dtype="<u4").tobytes())


def chained_trace(R, S, L, sel_pages, groups, seed=0, short=()):
    """Chained-hash-like ids: requests of a group share the ids of a prefix."""
    rng = np.random.default_rng(seed)
    bpp = 4
    prefix = {g: rng.integers(0, 2**32, size=64, dtype=np.uint64) for g in range(groups)}
    recs = []
    for r in range(R):
        own = rng.integers(0, 2**32, size=64, dtype=np.uint64)
        pool = np.concatenate([prefix[r % groups], own]).astype(np.uint32)
        rr = []
        for s in range(S):
            ls = []
            for l in range(L):
                pages = rng.choice(len(pool) // bpp, size=sel_pages, replace=False)
                ids = [int(pool[p * bpp + i]) for p in sorted(pages) for i in range(bpp)]
                if (r, s, l) in short:
                    ids = ids[:bpp]
                ls.append(ids)
            rr.append(ls)
        recs.append(rr)
    return recs


def test_known_answer_renaming(tmp_path):
    p = tmp_path / "t.bin"
    recs = [[[[0xDEADBEEF, 5, 0xDEADBEEF, 9, 7, 7, 5, 0]]], [[[9, 1, 2, 3, 0xDEADBEEF, 1, 1, 1]]]]
    write_fmt1(p, recs, R=2, S=1, L=1, sel_pages=2)
    info, ids = F.trace_load(str(p))
    want = np.array([[0, 1, 0, 2, 3, 3, 1, 4], [2, 5, 6, 7, 0, 5, 5, 5]], np.uint32)
    assert np.array_equal(ids.reshape(2, 8), want)
    assert info["unique_blocks"] == 8 and info["sel_blocks"] == 8
    assert info["max_blocks_per_req"] == 5  # request 0: deadbeef, 5, 9, 7, 0
    assert (info["requests"], info["steps"], info["layers"], info["page_tokens"],
            info["block_tokens"], info["kv_heads"], info["head_dim"], info["sel_pages"]) == \
        (2, 1, 1, 16, 4, 4, 128, 2)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_reader_matches_oracle(tmp_path, seed):
    R, S, L, SP = 6, 5, 3, 4
    recs = chained_trace(R, S, L, SP, groups=2, seed=seed)
    p = tmp_path / "t.bin"
    write_fmt1(p, recs, R, S, L, sel_pages=SP)
    info, ids = F.trace_load(str(p))
    hdr, oids, uniq, maxr = O.trace_load(str(p))
    assert np.array_equal(ids, oids)
    assert info["unique_blocks"] == uniq and info["max_blocks_per_req"] == maxr
    assert info["short_records"] == 0
    # renaming is a bijection that preserves equality of raw ids
    raw = np.array(recs, np.uint64).reshape(-1)
    d = ids.reshape(-1)
    assert len(np.unique(d)) == len(np.unique(raw))
    for v in np.unique(raw)[:50]:
        assert len(np.unique(d[raw == v])) == 1
    # first appearances come in order 0, 1, 2, ...
    _, first = np.unique(d, return_index=True)
    assert np.all(np.diff(first) > 0)


def test_short_records(tmp_path):
    R, S, L, SP = 3, 2, 2, 2
    recs = chained_trace(R, S, L, SP, groups=1, seed=4, short=[(1, 0, 1), (2, 1, 0)])
    p = tmp_path / "t.bin"
    write_fmt1(p, recs, R, S, L, sel_pages=SP)
    with pytest.raises(F.FerryError, match="4 ids at \\(r=1, s=0, l=1\\), expected 8"):
        F.trace_load(str(p), strict=True)
    info, ids = F.trace_load(str(p), strict=False)
    assert info["short_records"] == 2
    assert np.all(ids[1, 0, 1, 4:] == F.EMPTY) and np.all(ids[1, 0, 1, :4] != F.EMPTY)
    hdr, oids, _, _ = O.trace_load(str(p), strict=False)
    assert np.array_equal(ids, oids)


@pytest.mark.parametrize("bad,match", [
    (dict(magic=b"FMT2"), "magic"),
    (dict(version=2), "version"),
    (dict(page_tokens=10), "multiple"),
    (dict(page_tokens=0), "multiple"),
])
def test_bad_headers_are_refused(tmp_path, bad, match):
    p = tmp_path / "t.bin"
    write_fmt1(p, [[[[1] * 8]]], R=1, S=1, L=1, **bad)
    with pytest.raises(F.FerryError, match=match):
        F.trace_load(str(p))
    with pytest.raises(ValueError):
        O.trace_load(str(p))


def test_truncated_and_oversized_records_are_refused(tmp_path):
    p = tmp_path / "t.bin"
    write_fmt1(p, [[[list(range(8))], [list(range(8))]]], R=1, S=2, L=1)
    raw = p.read_bytes()
    for cut, match in [(20, "truncated header"), (len(raw) - 3, "truncated payload"),
                       (len(raw) - 34, "truncated payload")]:
        q = tmp_path / f"c{cut}.bin"
        q.write_bytes(raw[:cut])
        with pytest.raises(F.FerryError, match=match):
            F.trace_load(str(q))
    write_fmt1(p, [[[list(range(9))]]], R=1, S=1, L=1)
    with pytest.raises(F.FerryError, match="more than 8"):
        F.trace_load(str(p), strict=False)
    with pytest.raises(F.FerryError, match="cannot open"):
        F.trace_load(str(tmp_path / "missing.bin"))


@pytest.mark.parametrize("seed", range(4))
def test_corrupted_files_load_or_refuse(tmp_path, seed):
    """Random truncations, bit flips, overwritten header fields and garbage:
    the reader either loads a trace of the header's shape or raises
    FerryError, and when it loads, the oracle's reader agrees."""
    rng = np.random.default_rng(seed)
    p = tmp_path / "t.bin"
    write_fmt1(p, chained_trace(3, 2, 2, 2, 2, seed=seed), R=3, S=2, L=2, sel_pages=2)
    raw = bytearray(p.read_bytes())
    for i in range(60):
        b = bytearray(raw)
        kind = i % 4
        if kind == 0:
            b = b[:int(rng.integers(0, len(b)))]
        elif kind == 1:
            for _ in range(int(rng.integers(1, 8))):
                j = int(rng.integers(0, len(b)))
                b[j] ^= 1 << int(rng.integers(0, 8))
        elif kind == 2:  # a header field (R, S, L, geometry or sel_pages) overwritten
            j = 8 + 4 * int(rng.integers(0, 8))
            b[j:j + 4] = struct.pack("<I", int(rng.choice([0, 1, 3, 7, 1 << 20, 0xFFFFFFFF])))
        else:
            b = bytearray(rng.integers(0, 256, int(rng.integers(0, 200)), dtype=np.uint8).tobytes())
        q = tmp_path / f"c{i}.bin"
        q.write_bytes(bytes(b))
        try:
            info, ids = F.trace_load(str(q), strict=False)
        except F.FerryError:
            continue
        assert ids.shape == (info["requests"], info["steps"], info["layers"], info["sel_blocks"])
        _, oids, _, _ = O.trace_load(str(q), strict=False)
        assert np.array_equal(ids, oids)
