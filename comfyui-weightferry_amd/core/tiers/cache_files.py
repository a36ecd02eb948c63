"""The SSD tier's cache file (core/tiers/cache_files.py of the reference: DiskBlockStore :104-187, new_cache_path /
cleanup_stale_cache_files / default_cache_dir :18-101).

When the streamed blocks' final bytes are not a model file's ranges (weights ComfyUI has patched -- LoRA baked --, a
model loaded from safetensors, any torch module), the capture writes the SSD tier's blocks into a cache file: block
i at i * stride, the stride its flat size rounded up to 4 KiB, each block flushed to the disk as it is written (so
the file does not sit in RAM as dirty pages -- RAM is what the SSD tier saves). The file belongs to the process
(wf_blocks_<pid>_<n>.bin); files of processes that no longer run are removed the first time a directory is used.

With WEIGHTFERRY_PERSIST_GB > 0 the file outlives the process (the reference's persistent SSD cache,
core/tiers/cache_files.py:227-287 and streaming/load_steps.py:1095-1160,1288-1306): it is named by a key of its
content -- the layout and the bytes of every block it holds (``content_key``) -- so a later load whose blocks have
the same final bytes reads the file instead of writing it again, and no change to the model, its LoRAs or the
layout can make it read stale bytes. The entry's metadata (``.json``) is written last, once every block is on the
drive: an entry without it, or whose data file has the wrong length, is written again. Entries beyond the cap are
removed, least recently used first."""
import itertools
import json
import os
import tempfile
import time

from ..env import get as _env_get
from .sources import FileBlockSource

_ALIGN_IO = 4096
_PREFIX = "wf_blocks_"
_COUNTER = itertools.count()
_CLEANED = set()


def align_up(n, a=_ALIGN_IO):
    return (n + a - 1) // a * a


def default_cache_dir():
    """WEIGHTFERRY_CACHE_DIR, else <temp directory>/weightferry_cache."""
    return _env_get("WEIGHTFERRY_CACHE_DIR") or os.path.join(tempfile.gettempdir(), "weightferry_cache")


def _pid_alive(pid):
    try:
        os.kill(pid, 0)
    except ProcessLookupError:
        return False
    except PermissionError:
        return True
    return True


def cleanup_stale_cache_files(directory):
    """Remove cache files of processes that no longer run; returns the bytes freed."""
    freed = 0
    try:
        names = os.listdir(directory)
    except OSError:
        return 0
    for name in names:
        if not (name.startswith(_PREFIX) and name.endswith(".bin")):
            continue
        try:
            pid = int(name[len(_PREFIX):].split("_")[0])
        except ValueError:
            continue
        if pid == os.getpid() or _pid_alive(pid):
            continue
        path = os.path.join(directory, name)
        try:
            size = os.path.getsize(path)
            os.remove(path)
            freed += size
        except OSError:
            pass
    return freed


def new_cache_path(directory):
    return os.path.join(directory, f"{_PREFIX}{os.getpid()}_{next(_COUNTER)}.bin")


class DiskBlockStore:
    """Fixed-stride block file: block i at i * stride (stride = block_bytes rounded up to 4 KiB). ``path``: write
    that file (a persistent entry's data file) instead of a new one of this process; ``keep``: leave the file on the
    drive when the store is deleted."""

    is_model_file = False

    def __init__(self, directory, block_bytes, n_blocks, path=None, keep=False):
        os.makedirs(directory, exist_ok=True)
        if directory not in _CLEANED:
            _CLEANED.add(directory)
            self.cleanup_freed = cleanup_stale_cache_files(directory)
        else:
            self.cleanup_freed = 0
        self.path = path or new_cache_path(directory)
        self.keep = keep
        self.block_bytes = int(block_bytes)
        self.stride = align_up(self.block_bytes)
        self.n_blocks = int(n_blocks)
        self._fd = os.open(self.path, os.O_RDWR | os.O_CREAT | os.O_TRUNC | getattr(os, "O_CLOEXEC", 0), 0o600)

    def write_block(self, i, cpu_uint8):
        """Write block i (a contiguous uint8 CPU tensor / array of block_bytes) and flush it to the disk."""
        if not 0 <= i < self.n_blocks:
            raise IndexError(f"block {i} of {self.n_blocks}")
        buf = memoryview(cpu_uint8.numpy() if hasattr(cpu_uint8, "numpy") else cpu_uint8).cast("B")
        if buf.nbytes != self.block_bytes:
            raise ValueError(f"block of {buf.nbytes} bytes for {self.block_bytes}")
        off, done = i * self.stride, 0
        while done < buf.nbytes:
            done += os.pwrite(self._fd, buf[done:], off + done)
        os.fsync(self._fd)

    def finalize(self):
        os.fsync(self._fd)

    def source(self):
        """The ring's view of the file: block i is [i * stride, + block_bytes)."""
        return FileBlockSource(self.path, [(i * self.stride, self.block_bytes) for i in range(self.n_blocks)])

    def delete(self):
        if self._fd is not None:
            os.close(self._fd)
            self._fd = None
        if self.keep:
            return
        try:
            os.remove(self.path)
        except OSError:
            pass

    def __del__(self):
        try:
            self.delete()
        except Exception:  # noqa: BLE001 -- interpreter shutdown
            pass


# ------------------------------------------------------------------------------------------ persistent entries
_ENTRY_PREFIX = "dit_persist_"


def persistent_dir(cache_dir=None):
    """Folder of the persistent entries: <cache_dir>/persistent for an explicit cache folder (the node's or
    WEIGHTFERRY_CACHE_DIR), else <XDG cache home or ~/.cache>/weightferry/persistent -- not the temp folder, which
    the host application may empty at every start."""
    base = cache_dir or _env_get("WEIGHTFERRY_CACHE_DIR")
    if not base:
        home = os.environ.get("XDG_CACHE_HOME") or os.path.join(os.path.expanduser("~"), ".cache")
        base = os.path.join(home, "weightferry")
    return os.path.join(base, "persistent")


def _hasher():
    try:
        import xxhash
        return xxhash.xxh3_128()
    except ImportError:  # the key only needs to be a strong content digest
        import hashlib
        return hashlib.blake2b(digest_size=16)


def content_key(layout, blocks):
    """Hex key of an SSD cache's content: ``layout`` (any repr-stable value: the parameter shapes and dtypes, their
    offsets, the block bytes, the positions) and, block after block, the raw bytes of each parameter (``blocks``: an
    iterable of parameter lists, CPU or GPU tensors)."""
    h = _hasher()
    h.update(repr(("wf-ssd-cache", 1, layout)).encode())
    for params in blocks:
        h.update(b"B")
        for p in params:
            t = p.detach()
            if t.device.type != "cpu":
                t = t.cpu()
            t = t.contiguous().reshape(-1)
            h.update(b"P%d:" % (t.numel() * t.element_size()))
            h.update(memoryview(t.view(_torch().uint8).numpy()))
    return h.hexdigest()


def _torch():
    import torch
    return torch


class PersistentEntry:
    """One persistent SSD cache entry: <dir>/dit_persist_<key>.bin (blocks at a 4 KiB stride) and its .json."""

    def __init__(self, directory, key, n_blocks, block_bytes):
        self.directory, self.key = directory, str(key)
        self.n_blocks, self.block_bytes = int(n_blocks), int(block_bytes)
        self.bin = os.path.join(directory, f"{_ENTRY_PREFIX}{self.key}.bin")
        self.json = self.bin[:-4] + ".json"
        self._store = None

    def complete(self):
        """The metadata names this key and layout, and the data file holds every block (the last one's padding may
        be missing). Marks the entry used (its metadata's time: least recently used entries go first)."""
        try:
            with open(self.json, encoding="utf-8") as f:
                meta = json.load(f)
            size = os.path.getsize(self.bin)
        except (OSError, ValueError):
            return False
        stride = align_up(self.block_bytes)
        ok = (isinstance(meta, dict) and meta.get("key") == self.key and meta.get("blocks") == self.n_blocks
              and meta.get("block_bytes") == self.block_bytes and self.n_blocks > 0
              and (self.n_blocks - 1) * stride + self.block_bytes <= size <= self.n_blocks * stride)
        if ok:
            try:
                os.utime(self.json)
            except OSError:
                pass
        return ok

    def source(self):
        stride = align_up(self.block_bytes)
        return FileBlockSource(self.bin, [(i * stride, self.block_bytes) for i in range(self.n_blocks)])

    def open_store(self):
        """A store writing the entry's data under a name of its own (<data file>.<pid>_<n>.tmp). The committed data
        file is never written in place: a process reading the entry meanwhile keeps its bytes, and two processes
        writing the same entry each write their own file. A write that stops part way leaves its temporary file,
        removed when the store is deleted (or, if the process died, by the next enforce_cap)."""
        os.makedirs(self.directory, exist_ok=True)
        self._store = DiskBlockStore(self.directory, self.block_bytes, self.n_blocks,
                                     path=f"{self.bin}.{os.getpid()}_{next(_COUNTER)}.tmp")
        return self._store

    def commit(self, cap_bytes):
        """The written data file renamed over the entry's (atomic: readers see the old file or the new one, whole),
        the metadata last (the entry is complete from here on), then older entries beyond ``cap_bytes`` removed.
        The store then refers to the entry's data file and leaves it on the drive. Returns the bytes removed."""
        store = self._store
        store.finalize()
        os.replace(store.path, self.bin)
        store.path, store.keep = self.bin, True
        tmp = f"{self.json}.{os.getpid()}_{next(_COUNTER)}.tmp"
        with open(tmp, "w", encoding="utf-8") as f:
            json.dump({"key": self.key, "blocks": self.n_blocks, "block_bytes": self.block_bytes,
                       "created": time.time()}, f)
            f.flush()
            os.fsync(f.fileno())
        os.replace(tmp, self.json)
        return enforce_cap(self.directory, cap_bytes, keep_key=self.key)


def enforce_cap(directory, cap_bytes, keep_key=None):
    """Remove persistent entries, least recently used first (an entry without metadata counts as the oldest),
    until the folder's entries hold at most ``cap_bytes``; ``keep_key`` is never removed. Returns the bytes
    removed."""
    try:
        names = os.listdir(directory)
    except OSError:
        return 0
    entries = {}
    for name in names:
        if not name.startswith(_ENTRY_PREFIX):
            continue
        if name.endswith(".tmp"):
            # an entry being written (<name>.<pid>_<n>.tmp): its writer renames or removes it; one left by a process
            # that no longer runs is removed here
            try:
                pid = int(name.rsplit(".", 2)[-2].split("_")[0])
            except ValueError:
                continue
            if pid != os.getpid() and not _pid_alive(pid):
                try:
                    os.remove(os.path.join(directory, name))
                except OSError:
                    pass
            continue
        key = name[len(_ENTRY_PREFIX):].split(".", 1)[0]
        path = os.path.join(directory, name)
        try:
            st = os.stat(path)
        except OSError:
            continue
        e = entries.setdefault(key, {"files": [], "used": -1.0})
        e["files"].append((path, st.st_size))
        if name.endswith(".json"):
            e["used"] = st.st_mtime
    total = sum(n for e in entries.values() for _, n in e["files"])
    removed = 0
    for key, e in sorted(entries.items(), key=lambda kv: kv[1]["used"]):
        if total <= cap_bytes:
            break
        if key == keep_key:
            continue
        for path, n in e["files"]:
            try:
                os.remove(path)
            except OSError:   # still there: it still counts
                continue
            total -= n
            removed += n
    return removed
