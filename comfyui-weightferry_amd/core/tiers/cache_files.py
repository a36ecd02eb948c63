"""The SSD tier's cache file (core/tiers/cache_files.py of the reference: DiskBlockStore :104-187, new_cache_path /
cleanup_stale_cache_files / default_cache_dir :18-101).

When the streamed blocks' final bytes are not a model file's ranges (weights ComfyUI has patched -- LoRA baked --, a
model loaded from safetensors, any torch module), the capture writes the SSD tier's blocks into a cache file: block
i at i * stride, the stride its flat size rounded up to 4 KiB, each block flushed to the disk as it is written (so
the file does not sit in RAM as dirty pages -- RAM is what the SSD tier saves). The file belongs to the process
(wf_blocks_<pid>_<n>.bin); files of processes that no longer run are removed the first time a directory is used."""
import itertools
import os
import tempfile

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
    """Fixed-stride block file: block i at i * stride (stride = block_bytes rounded up to 4 KiB)."""

    is_model_file = False

    def __init__(self, directory, block_bytes, n_blocks):
        os.makedirs(directory, exist_ok=True)
        if directory not in _CLEANED:
            _CLEANED.add(directory)
            self.cleanup_freed = cleanup_stale_cache_files(directory)
        else:
            self.cleanup_freed = 0
        self.path = new_cache_path(directory)
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
        try:
            os.remove(self.path)
        except OSError:
            pass

    def __del__(self):
        try:
            self.delete()
        except Exception:  # noqa: BLE001 -- interpreter shutdown
            pass
