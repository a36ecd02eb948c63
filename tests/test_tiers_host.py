"""The SSD tier's host side on the CPU: the drive probe that sizes the reader ring (the reference's
core/tiers/disk_io.py:165-209, used by plan_tiers, core/tiers/plan.py:60-150) and the persistent cache entries
(core/tiers/cache_files.py:227-287, streaming/load_steps.py:1095-1160,1288-1306 of the reference), here keyed by
the cached blocks' content."""
import json
import os
import time

import pytest
import torch

from conftest import sub

disk_io = sub("core.tiers.disk_io")
plan = sub("core.tiers.plan")
cf = sub("core.tiers.cache_files")
ls = sub("streaming.load_steps")


def test_probe_measures_and_remembers(tmp_path, monkeypatch):
    d = str(tmp_path / "drive")
    p = disk_io.probe_disk(d, size_mb=8, chunk_mb=1)
    assert p["gbps"] > 0 and p["threads"] in (1, 2, 4) and sorted(p["by_threads"]) == [1, 2, 4]
    assert p["gbps"] == max(p["by_threads"].values())
    assert not os.path.exists(os.path.join(d, "weightferry_disk_probe.bin"))      # scratch file removed
    with open(os.path.join(d, "weightferry_disk_probe.json")) as f:
        kept = json.load(f)
    assert kept["size_mb"] == 8 and kept["chunk_mb"] == 1

    def no_read(*a, **k):
        raise AssertionError("measured again")
    monkeypatch.setattr(disk_io, "timed_read", no_read)
    assert disk_io.probe_disk(d, size_mb=8, chunk_mb=1) == p                     # from the kept result
    # other parameters, an old result or a damaged file: measured again
    for bad in ({"size_mb": 16}, {"chunk_mb": 2}, {"thread_counts": (1, 2)}):
        with pytest.raises(AssertionError, match="measured again"):
            disk_io.probe_disk(d, **dict({"size_mb": 8, "chunk_mb": 1}, **bad))
    kept["time"] = time.time() - 8 * 24 * 3600
    with open(os.path.join(d, "weightferry_disk_probe.json"), "w") as f:
        json.dump(kept, f)
    with pytest.raises(AssertionError, match="measured again"):
        disk_io.probe_disk(d, size_mb=8, chunk_mb=1)
    with open(os.path.join(d, "weightferry_disk_probe.json"), "w") as f:
        f.write("{not json")
    with pytest.raises(AssertionError, match="measured again"):
        disk_io.probe_disk(d, size_mb=8, chunk_mb=1)


def test_timed_read_covers_the_file(tmp_path):
    path = str(tmp_path / "f.bin")
    with open(path, "wb") as f:
        f.write(os.urandom(3 << 20))
    for threads in (1, 2, 4):
        gbps, _ = disk_io.timed_read(path, 3 << 20, 1 << 20, threads)
        assert gbps > 0
    with pytest.raises(OSError):
        disk_io.timed_read(path, 5 << 20, 1 << 20, 2)                           # past the end: a short read


def test_plan_takes_depth_and_threads_from_the_probe(tmp_path, monkeypatch):
    GB = 1 << 30
    calls = []

    def fake_probe(directory, size_mb=512, **k):
        calls.append((directory, size_mb))
        return {"gbps": 6.0, "threads": 2, "by_threads": {1: 3.0, 2: 6.0, 4: 5.0}, "direct": True}
    monkeypatch.setattr(disk_io, "probe_disk", fake_probe)
    monkeypatch.setenv("WEIGHTFERRY_DISK_PROBE_MB", "64")
    p = plan.plan_tiers(40, 200 << 20, ram_budget_bytes=4 * GB, disk_dir=str(tmp_path), compute_ms_per_block=5.0)
    assert calls == [(str(tmp_path), 64)]
    # 200 MiB at 6 GB/s = 35 ms per block against 5 ms of compute: ceil(7) + 2 = 9 -> 8 buffers
    assert p["ring_threads"] == 2 and p["disk_read_gbps"] == 6.0 and p["ring_depth"] == 8
    assert p["ram_blocks"] == (4 * GB - 8 * (200 << 20)) // (200 << 20)
    monkeypatch.setenv("WEIGHTFERRY_DISK_THREADS", "4")
    p = plan.plan_tiers(40, 200 << 20, ram_budget_bytes=4 * GB, disk_dir=str(tmp_path))
    assert p["ring_threads"] == 4 and p["disk_read_gbps"] == 5.0 and p["ring_depth"] == 4
    # everything fits in RAM: no probe
    calls.clear()
    assert plan.plan_tiers(4, 1 << 20, ram_budget_bytes=GB, disk_dir=str(tmp_path))["disk_blocks"] == 0
    assert calls == []

    def failing(*a, **k):
        raise OSError("read-only")
    monkeypatch.setattr(disk_io, "probe_disk", failing)
    p = plan.plan_tiers(40, 200 << 20, ram_budget_bytes=4 * GB, disk_dir=str(tmp_path))
    assert p["disk_error"] == "read-only" and p["ring_depth"] == 4 and p["disk_read_gbps"] is None


def test_content_key_follows_every_byte_and_the_layout():
    torch.manual_seed(0)
    blocks = [[torch.randn(300), torch.randn(7, 5).to(torch.bfloat16)] for _ in range(3)]
    k = cf.content_key(("layout", 1), blocks)
    assert k == cf.content_key(("layout", 1), [[t.clone() for t in b] for b in blocks])
    assert k != cf.content_key(("layout", 2), blocks)
    changed = [[t.clone() for t in b] for b in blocks]
    changed[2][1].view(torch.int16)[3, 4] ^= 1                                   # one bit of the last block
    assert k != cf.content_key(("layout", 1), changed)
    assert k != cf.content_key(("layout", 1), blocks[:2])                        # one block fewer
    # the bytes of a parameter, not only its values: an empty tensor still counts as a parameter
    assert cf.content_key(0, [[torch.zeros(0)]]) != cf.content_key(0, [[]])


def test_persistent_entry_is_complete_only_after_commit(tmp_path):
    e = cf.PersistentEntry(str(tmp_path), "k1", 3, 5000)
    assert not e.complete()
    store = e.open_store()
    for i in range(3):
        store.write_block(i, torch.full((5000,), i, dtype=torch.uint8))
    store.finalize()
    assert not e.complete()                                                      # no metadata yet
    e.commit(cap_bytes=1 << 30)
    assert e.complete()
    store.delete()
    assert os.path.exists(e.bin)                                                 # kept on the drive
    src = e.source()
    assert src.ranges == [(0, 5000), (4096 * 2, 5000), (4096 * 4, 5000)]
    assert not cf.PersistentEntry(str(tmp_path), "k1", 4, 5000).complete()       # another layout
    assert not cf.PersistentEntry(str(tmp_path), "k1", 3, 4000).complete()
    with open(e.bin, "r+b") as f:                                                # a data file cut short
        f.truncate(2 * 8192)
    assert not e.complete()
    # a rewrite goes to a file of its own: the committed data file is not cut while another process may read it, and
    # a rewrite abandoned part way removes its file and leaves the entry as it was
    e2 = cf.PersistentEntry(str(tmp_path), "k1", 3, 5000)
    size = os.path.getsize(e.bin)
    st2 = e2.open_store()
    assert st2.path != e.bin and os.path.getsize(e.bin) == size
    st2.write_block(0, torch.full((5000,), 9, dtype=torch.uint8))
    tmp_file = st2.path
    st2.delete()
    assert not os.path.exists(tmp_file) and os.path.getsize(e.bin) == size and os.path.exists(e.json)


def test_two_writers_of_one_entry(tmp_path):
    # two loads miss the same entry and both write it: each writes its own file and renames it into place, so a
    # reader that opened the first commit's file keeps whole bytes, and the entry is complete after either commit
    a = cf.PersistentEntry(str(tmp_path), "k2", 2, 5000)
    b = cf.PersistentEntry(str(tmp_path), "k2", 2, 5000)
    sa, sb = a.open_store(), b.open_store()
    for st in (sa, sb):
        for i in range(2):
            st.write_block(i, torch.full((5000,), i + 1, dtype=torch.uint8))
    a.commit(cap_bytes=1 << 30)
    assert a.complete() and sa.path == a.bin
    reader = open(a.bin, "rb")
    b.commit(cap_bytes=1 << 30)
    assert b.complete()
    reader.seek(8192)                                                            # block 1 (4 KiB stride)
    assert reader.read(5000) == bytes([2]) * 5000
    reader.close()
    sa.delete()
    sb.delete()
    assert os.path.exists(a.bin) and not [n for n in os.listdir(tmp_path) if n.endswith(".tmp")]


def test_cap_removes_a_dead_writers_file(tmp_path):
    live = tmp_path / f"dit_persist_k3.bin.{os.getpid()}_0.tmp"
    dead = tmp_path / "dit_persist_k4.bin.999999999_0.tmp"
    for f in (live, dead):
        f.write_bytes(b"\0" * 100)
    cf.enforce_cap(str(tmp_path), 0)
    assert live.exists() and not dead.exists()


def _entry(d, key, nbytes, used):
    with open(os.path.join(d, f"dit_persist_{key}.bin"), "wb") as f:
        f.write(b"\0" * nbytes)
    if used is not None:
        j = os.path.join(d, f"dit_persist_{key}.json")
        with open(j, "w") as f:
            f.write("{}")
        os.utime(j, (used, used))


def test_cap_removes_least_recently_used_entries(tmp_path):
    d = str(tmp_path)
    now = time.time()
    _entry(d, "a", 1000, now - 300)
    _entry(d, "b", 1000, now - 100)
    _entry(d, "c", 1000, None)                                                   # no metadata: oldest
    _entry(d, "d", 1000, now - 200)
    with open(os.path.join(d, "other.bin"), "wb") as f:                          # not an entry: left alone
        f.write(b"x" * 5000)
    removed = cf.enforce_cap(d, 2100, keep_key="a")
    names = sorted(os.listdir(d))
    # c goes first, then d (a is kept although older); b and a remain
    assert "dit_persist_c.bin" not in names and "dit_persist_d.bin" not in names
    assert "dit_persist_a.bin" in names and "dit_persist_b.bin" in names and "other.bin" in names
    assert removed == 1000 + 1002                                                # c, then d's data and metadata


def test_ssd_cache_written_once_then_reused(tmp_path, monkeypatch):
    # the same blocks' bytes in a later load read the kept entry; other bytes make a new entry
    monkeypatch.setenv("WEIGHTFERRY_PERSIST_GB", "1")
    common = sub("streaming.common")
    torch.manual_seed(3)
    blocks = [torch.nn.Linear(64, 32).requires_grad_(False) for _ in range(5)]
    specs = common._specs(blocks[0])
    offsets, flat = common._flat_layout(specs)
    ssd = {"cache_dir": str(tmp_path)}
    src1, store1 = ls._ssd_cache(blocks, [1, 3, 4], specs, offsets, flat, ssd)
    assert store1 is not None and store1.keep and os.path.dirname(src1.path) == str(tmp_path / "persistent")
    raw = open(src1.path, "rb").read()
    stage = torch.zeros(flat, dtype=torch.uint8)
    for k, s in enumerate([1, 3, 4]):
        stage.zero_()
        for p, v in zip(blocks[s].parameters(), common._views(stage, specs, offsets)):
            v.copy_(p.data)
        o, n = src1.ranges[k]
        assert raw[o:o + n] == bytes(stage.numpy())
    store1.delete()

    def no_write(*a, **k):
        raise AssertionError("written again")
    monkeypatch.setattr(cf.DiskBlockStore, "write_block", no_write)
    src2, store2 = ls._ssd_cache(blocks, [1, 3, 4], specs, offsets, flat, ssd)
    assert store2 is None and src2.path == src1.path and src2.ranges == src1.ranges
    blocks[3].weight[0, 0] += 1
    with pytest.raises(AssertionError, match="written again"):
        ls._ssd_cache(blocks, [1, 3, 4], specs, offsets, flat, ssd)
    # without the flag (and with writes back): a cache file of this process, removed at teardown
    monkeypatch.undo()
    src3, store3 = ls._ssd_cache(blocks, [0], specs, offsets, flat, ssd)
    assert not store3.keep and os.path.basename(src3.path).startswith("wf_blocks_")
    store3.delete()
    assert not os.path.exists(src3.path)


def test_read_packed_assembles_pieces(tmp_path):
    sources = sub("core.tiers.sources")
    path = str(tmp_path / "f.bin")
    data = os.urandom(10000)
    with open(path, "wb") as f:
        f.write(data)
    # block 0: bytes 100..399 of the file at packed 0, 5000..5099 at packed 512 (padding 300..511 reads as zero)
    src = sources.PieceFileSource(path, [[(100, 300, 0), (5000, 100, 512)], [(0, 10, 0)]])
    out = bytearray(700)
    sources.read_packed(src, 0, 0, 700, out)
    assert out[:300] == data[100:400] and out[300:512] == bytes(212) and out[512:612] == data[5000:5100]
    out = bytearray(20)
    sources.read_packed(src, 0, 505, 20, out)
    assert out[:7] == bytes(7) and out[7:] == data[5000:5013]
