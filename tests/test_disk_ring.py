"""The SSD tier's native reader ring (wf_ring_*) in host mode (plain aligned buffers, acquire / release), on the
CPU: every block's bytes equal the file's ranges over several cycles, for one-piece and multi-piece blocks at
unaligned offsets, several depths and reader threads, with and without O_DIRECT; the cyclic order is enforced;
read failures reach the consumer; resync restarts the cycle (the contract of DiskRing, core/tiers/sources.py:
165-355 of the reference, and of its FileBlockSource / PieceFileSource)."""
import os

import numpy as np
import pytest

from conftest import sub

src = sub("core.tiers.sources")
native = sub("_native")
plan = sub("core.tiers.plan")


@pytest.fixture
def blob(tmp_path):
    rng = np.random.default_rng(3)
    data = rng.integers(0, 256, 3 << 20, dtype=np.uint8)
    p = tmp_path / "blob.bin"
    p.write_bytes(data.tobytes())
    return str(p), data


def expect_block(data, pieces):
    n = max(d + k for _, k, d in pieces)
    out = np.zeros(n, dtype=np.uint8)
    for o, k, d in pieces:
        out[d:d + k] = data[o:o + k]
    return out


def consume(ring, source, data, cycles, order=None):
    pcs = source.pieces()
    for c in range(cycles):
        for d in range(source.n_blocks):
            view, slot = ring.acquire(d)
            want = expect_block(data, pcs[d])
            got = view.numpy()
            assert got.size == want.size
            # multi-piece blocks: only the pieces' bytes are defined (gaps between pieces stay as they were)
            for o, k, dd in pcs[d]:
                assert np.array_equal(got[dd:dd + k], data[o:o + k]), (c, d)
            ring.release(slot)


@pytest.mark.parametrize("depth,threads,direct", [(1, 1, False), (2, 1, True), (3, 2, True), (4, 4, False)])
def test_one_piece_blocks_over_cycles(blob, depth, threads, direct):
    path, data = blob
    ranges = [(5, 100_000), (131_072, 262_144), (700_001, 4097), (1_000_000, 1_048_576), (3 * (1 << 20) - 999, 999)]
    source = src.FileBlockSource(path, ranges)
    ring = src.DiskRing(source, depth=depth, pin=False, threads=threads, direct=direct)
    try:
        consume(ring, source, data, 3)
        st = ring.stats()
        assert st["reads"] >= 3 * len(ranges) and st["bytes"] > 0
    finally:
        ring.close()


@pytest.mark.parametrize("direct", [False, True])
def test_multi_piece_blocks(blob, direct):
    path, data = blob
    pieces = [
        [(10, 300, 0), (9000, 5000, 512), (200_003, 70_000, 6000)],
        [(4096, 4096, 0), (8192, 4096, 4096)],
        [(3 * (1 << 20) - 1000, 1000, 100), (1, 1, 2000)],
    ]
    source = src.PieceFileSource(path, pieces)
    ring = src.DiskRing(source, depth=2, pin=False, threads=2, direct=direct)
    try:
        consume(ring, source, data, 2)
    finally:
        ring.close()


def test_merge_pieces_joins_file_adjacent_runs():
    assert src.merge_pieces([(1000, 10, 0), (1256, 20, 256), (1600, 4, 600)]) == [(1000, 604, 0)]
    assert src.merge_pieces([(1000, 10, 0), (1300, 20, 256)]) == [(1000, 10, 0), (1300, 20, 256)]


def test_order_is_enforced(blob):
    path, data = blob
    source = src.FileBlockSource(path, [(0, 4096), (4096, 4096), (8192, 4096)])
    ring = src.DiskRing(source, depth=2, pin=False)
    try:
        with pytest.raises(native.NativeError, match="out of sync"):
            ring.acquire(1)
        view, slot = ring.acquire(0)
        with pytest.raises(native.NativeError, match="acquired last"):
            ring.release((slot + 1) % 2)
        ring.release(slot)
        view, slot = ring.acquire(1)
        ring.release(slot)
    finally:
        ring.close()


def test_resync_restarts_the_cycle(blob):
    path, data = blob
    source = src.FileBlockSource(path, [(i * 8192, 8192) for i in range(5)])
    ring = src.DiskRing(source, depth=3, pin=False, threads=2)
    try:
        for d in range(2):
            v, s = ring.acquire(d)
            ring.release(s)
        ring.resync()
        consume(ring, source, data, 2)
    finally:
        ring.close()


def test_read_failure_reaches_the_consumer(tmp_path):
    p = tmp_path / "short.bin"
    p.write_bytes(bytes(1 << 16))
    source = src.FileBlockSource(str(p), [(0, 1 << 15), (1 << 15, 1 << 15)])
    ring = src.DiskRing(source, depth=2, pin=False)
    try:
        for d in range(2):
            v, s = ring.acquire(d)
            ring.release(s)
        os.truncate(p, 1 << 15)          # the file shrinks under the ring: block 1 is cut short
        ring.resync()
        v, s = ring.acquire(0)
        ring.release(s)
        with pytest.raises(native.NativeError, match="end of file"):
            ring.acquire(1)
    finally:
        ring.close()


def test_open_rejects_ranges_outside_the_file(blob):
    path, data = blob
    with pytest.raises(native.NativeError, match="outside the file"):
        src.DiskRing(src.FileBlockSource(path, [(len(data) - 10, 11)]), pin=False)
    with pytest.raises(native.NativeError, match="overlap"):
        src.DiskRing(src.PieceFileSource(path, [[(0, 100, 0), (500, 100, 50)]]), pin=False)
    with pytest.raises(native.NativeError):
        src.DiskRing(src.FileBlockSource(path + ".missing", [(0, 10)]), pin=False)


def test_ssd_positions():
    assert plan.ssd_positions(40, 0) == []
    assert plan.ssd_positions(10, 3, "tail") == [7, 8, 9]
    assert plan.ssd_positions(4, 9) == [0, 1, 2, 3]
    pos = plan.ssd_positions(40, 10)
    assert pos == [3, 7, 11, 15, 19, 23, 27, 31, 35, 39]
    for n in range(1, 41):
        p = plan.ssd_positions(40, n)
        assert len(p) == n and p == sorted(set(p)) and p[-1] == 39 and p[0] >= 0


@pytest.mark.parametrize("direct", [False, True])
def test_pieces_larger_than_the_read_chunk(tmp_path, direct):
    # O_DIRECT reads go through an 8 MiB scratch buffer: a 17 MiB piece at an unaligned offset takes three chunks
    rng = np.random.default_rng(11)
    data = rng.integers(0, 256, 40 << 20, dtype=np.uint8)
    p = tmp_path / "big.bin"
    p.write_bytes(data.tobytes())
    pieces = [[(12_345, 17 << 20, 0), ((20 << 20) + 3, 1 << 20, (17 << 20) + 256)],
              [((40 << 20) - (9 << 20) - 1, 9 << 20, 0)]]
    source = src.PieceFileSource(str(p), pieces)
    ring = src.DiskRing(source, depth=2, pin=False, threads=2, direct=direct)
    try:
        consume(ring, source, data, 2)
    finally:
        ring.close()


def test_cache_file_store_round_trip_and_stale_cleanup(tmp_path):
    cf = sub("core.tiers.cache_files")
    d = str(tmp_path / "cache")
    os.makedirs(d)
    dead = 4_194_301
    while True:                                    # a pid that no process has
        try:
            os.kill(dead, 0)
            dead -= 1
        except ProcessLookupError:
            break
        except PermissionError:
            dead -= 1
    stale = os.path.join(d, f"wf_blocks_{dead}_0.bin")
    mine = os.path.join(d, f"wf_blocks_{os.getpid()}_999.bin")
    for p in (stale, mine):
        open(p, "wb").write(b"x" * 10)
    rng = np.random.default_rng(2)
    block_bytes = 3 * 4096 + 123
    store = cf.DiskBlockStore(d, block_bytes, 4)
    assert not os.path.exists(stale) and os.path.exists(mine) and store.cleanup_freed == 10
    data = [rng.integers(0, 256, block_bytes, dtype=np.uint8) for _ in range(4)]
    for i, b in enumerate(data):
        store.write_block(i, b)
    store.finalize()
    assert os.path.getsize(store.path) == 3 * store.stride + block_bytes and store.stride % 4096 == 0
    ring = src.DiskRing(store.source(), depth=2, pin=False, threads=2, direct=True)
    try:
        for c in range(2):
            for i in range(4):
                v, s = ring.acquire(i)
                assert np.array_equal(v.numpy(), data[i])
                ring.release(s)
    finally:
        ring.close()
    path = store.path
    store.delete()
    assert not os.path.exists(path)


def test_plan_tiers():
    GB = 1 << 30
    p = plan.plan_tiers(40, GB // 5, ram_budget_bytes=100 * GB)
    assert p == {"ram_blocks": 40, "disk_blocks": 0, "ring_depth": 0, "ring_threads": 1, "budget": 100 * GB,
                 "ssd_bound": False, "disk_read_gbps": None, "disk_error": None}
    # 4 GB for 200 MB blocks: a ring of 4 (default) takes 0.8 GB, 16 blocks fit in the rest
    p = plan.plan_tiers(40, 200 << 20, ram_budget_bytes=4 * GB)
    assert p["ring_depth"] == 4 and p["ram_blocks"] == (4 * GB - 4 * (200 << 20)) // (200 << 20) == 16
    assert p["disk_blocks"] == 24
    # the ring covers one read with compute: 200 MB at 5 GB/s = 42 ms over 4 ms of compute -> 8 (the cap)
    p = plan.plan_tiers(40, 200 << 20, ram_budget_bytes=4 * GB, disk_gbps=5.0, compute_ms_per_block=4.0)
    assert p["ring_depth"] == 8 and p["ssd_bound"]
    p = plan.plan_tiers(40, 200 << 20, ram_budget_bytes=4 * GB, disk_gbps=5.0, compute_ms_per_block=40.0)
    assert p["ring_depth"] == 4 and not p["ssd_bound"]
    # a budget below the ring: depth drops to 2, nothing in RAM
    p = plan.plan_tiers(40, 200 << 20, ram_budget_bytes=300 << 20)
    assert p["ring_depth"] == 2 and p["ram_blocks"] == 0 and p["disk_blocks"] == 40
    # automatic budget: the available RAM minus the margin
    p = plan.plan_tiers(2, 1, ram_margin_bytes=0)
    assert p["ram_blocks"] == 2
