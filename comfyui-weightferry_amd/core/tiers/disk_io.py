"""Read rate of the drive that holds the SSD tier, measured once and remembered (the role of the reference's
probe_disk, core/tiers/disk_io.py:165-209): it sizes the reader ring's depth and thread count (core.tiers.plan).

The probe writes a scratch file of ``size_mb`` MiB into the directory, flushes it to the drive, then reads it back
with 1, 2 and 4 threads (each thread a contiguous share, ``chunk_mb`` MiB per read) the way the ring reads: O_DIRECT
into page-aligned buffers, so the page cache the write just filled is not what gets measured. A file system that
refuses O_DIRECT (tmpfs, some network mounts) is read through the page cache after asking the kernel to drop the
file's pages; the result records which ("direct"). The figures are kept in ``weightferry_disk_probe.json`` in the
directory for ``max_age_s`` (a week) and reused while the probe's parameters are the same."""
import json
import mmap
import os
import threading
import time

_CACHE_NAME = "weightferry_disk_probe.json"
_SCRATCH_NAME = "weightferry_disk_probe.bin"
_VERSION = 1
MB = 1024 ** 2


def _open_read(path):
    """(fd, direct): O_DIRECT where the file system takes it."""
    flag = getattr(os, "O_DIRECT", 0)
    if flag:
        try:
            return os.open(path, os.O_RDONLY | flag), True
        except OSError:
            pass
    fd = os.open(path, os.O_RDONLY)
    if hasattr(os, "posix_fadvise"):
        os.posix_fadvise(fd, 0, 0, os.POSIX_FADV_DONTNEED)
    return fd, False


def _read_share(path, start, end, chunk, errors, direct_seen):
    fd = None
    try:
        fd, direct = _open_read(path)
        direct_seen.append(direct)
        buf = mmap.mmap(-1, chunk)              # page-aligned, as O_DIRECT needs
        try:
            off = start
            while off < end:
                n = os.preadv(fd, [memoryview(buf)[:min(chunk, end - off)]], off)
                if n <= 0:
                    raise OSError(f"short read at {off} of {path}")
                off += n
        finally:
            buf.close()
    except BaseException as exc:  # noqa: BLE001 -- handed to the caller
        errors.append(exc)
    finally:
        if fd is not None:
            os.close(fd)


def timed_read(path, nbytes, chunk, threads):
    """GB/s of reading [0, nbytes) of ``path`` with ``threads`` threads, each a contiguous chunk-aligned share;
    returns (GB/s, direct)."""
    per = -(-nbytes // threads)
    per = -(-per // chunk) * chunk
    errors, direct_seen, workers = [], [], []
    for t in range(threads):
        a, b = t * per, min(nbytes, (t + 1) * per)
        if a < b:
            workers.append(threading.Thread(target=_read_share, args=(path, a, b, chunk, errors, direct_seen),
                                            daemon=True))
    t0 = time.perf_counter()
    for w in workers:
        w.start()
    for w in workers:
        w.join()
    dt = time.perf_counter() - t0
    if errors:
        raise errors[0]
    return nbytes / dt / 1e9, all(direct_seen)


def _cached(path, size_mb, chunk_mb, thread_counts, max_age_s):
    try:
        with open(path, encoding="utf-8") as f:
            c = json.load(f)
        by = {int(k): float(v) for k, v in c["by_threads"].items()}
    except (OSError, ValueError, KeyError, TypeError, AttributeError):
        return None
    if (c.get("version") != _VERSION or c.get("size_mb") != size_mb or c.get("chunk_mb") != chunk_mb
            or sorted(by) != sorted(thread_counts) or not 0 <= time.time() - float(c.get("time", 0)) < max_age_s):
        return None
    return by, bool(c.get("direct"))


def _result(by, direct):
    best = max(sorted(by), key=lambda n: by[n])
    return {"gbps": by[best], "threads": best, "by_threads": dict(by), "direct": direct}


def probe_disk(directory, size_mb=512, chunk_mb=32, thread_counts=(1, 2, 4), max_age_s=7 * 24 * 3600):
    """{"gbps": best read GB/s, "threads": its thread count, "by_threads": {threads: GB/s}, "direct": O_DIRECT used}
    for the drive holding ``directory`` (created if missing); measured at most once per ``max_age_s``."""
    os.makedirs(directory, exist_ok=True)
    cache = os.path.join(directory, _CACHE_NAME)
    hit = _cached(cache, size_mb, chunk_mb, tuple(thread_counts), max_age_s)
    if hit is not None:
        return _result(*hit)
    scratch = os.path.join(directory, _SCRATCH_NAME)
    block = os.urandom(MB)
    try:
        with open(scratch, "wb") as f:
            for _ in range(size_mb):
                f.write(block)
            f.flush()
            os.fsync(f.fileno())
        by, direct = {}, True
        for n in thread_counts:
            gbps, d = timed_read(scratch, size_mb * MB, chunk_mb * MB, int(n))
            by[int(n)] = round(gbps, 3)
            direct = direct and d
    finally:
        try:
            os.remove(scratch)
        except OSError:
            pass
    try:
        with open(cache, "w", encoding="utf-8") as f:
            json.dump({"version": _VERSION, "by_threads": by, "size_mb": size_mb, "chunk_mb": chunk_mb,
                       "time": time.time(), "direct": direct}, f)
    except OSError:  # only a shortcut for the next load
        pass
    return _result(by, direct)
