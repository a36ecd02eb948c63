// SSD tier: a ring of host buffers that reader threads fill with streamed blocks read from a file (the model file
// itself, or a cache file), in cyclic block order, and -- in the GPU mode -- an uploader thread that copies each
// block into its GPU slot on the caller's copy stream. The role of the reference's DiskRing
// (core/tiers/sources.py:165-355), FileBlockSource / PieceFileSource (:87-152) and _SsdUploader
// (streaming/ssd_uploader.py:17-120), as one native object.
//
// Blocks are lists of pieces (file offset, bytes, offset in the packed block); each piece lands at its offset in
// the buffer. With O_DIRECT (flag WF_RING_DIRECT) reads bypass the page cache: each piece's 4 KiB aligned superset
// is read in 8 MiB chunks into the reader's aligned scratch buffer and copied to its place; where the file system
// refuses O_DIRECT the reader falls back to ordinary reads, straight into the buffer.
//
// Order: the ring reads positions 0, 1, 2, ... (block = position % n_blocks) into buffer position % depth, and the
// consumer takes blocks in the same order -- the forward passes consume the SSD-tier blocks in order, so reads run
// on into the next pass. A buffer is refilled only after the copy out of it has finished (its event).
//
// Consumers: acquire / release from one host thread (host mode, or the caller does its own copy), or submit /
// wait (GPU mode: the uploader thread waits for the block, makes the copy stream wait for the slot-free event,
// copies, records the done event and the buffer's copy event, and returns the buffer to the readers). The two
// consumer forms are not mixed on one ring.
#include <errno.h>
#include <fcntl.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <time.h>
#include <unistd.h>

#include <algorithm>
#include <condition_variable>
#include <deque>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "host_common.h"

namespace wf {
namespace {

constexpr int64_t kAlign = 4096;
int64_t align_down(int64_t v) { return v / kAlign * kAlign; }
int64_t align_up(int64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

double now_s() {
    timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec + ts.tv_nsec * 1e-9;
}

struct Piece { int64_t off, len, dst; };

struct Job {
    int64_t block, ticket;
    void* dst;
    int64_t dst_bytes;
    hipEvent_t wait_ev, done_ev;
    hipStream_t stream;
};

struct Slot {
    int64_t pos = -1;            // position whose bytes the buffer holds (valid when ready)
    int64_t nbytes = 0;
    bool ready = false;
    hipEvent_t copy_ev = nullptr;  // GPU mode: the copy out of this buffer
    bool copy_pending = false;
};

struct Ring {
    std::string path;
    int device = 0;
    bool pinned = false, direct = false;
    int64_t n_blocks = 0;
    std::vector<int64_t> pstart;
    std::vector<Piece> pieces;
    std::vector<int64_t> block_bytes;
    int64_t buf_bytes = 0;
    int depth = 0, n_threads = 0;
    uint8_t* bufs = nullptr;
    std::vector<Slot> slots;

    std::mutex m;
    std::condition_variable cv_read, cv_ready, cv_job, cv_done;
    std::deque<std::pair<int64_t, int>> reads;   // (position, slot)
    int64_t req = 0, cons = 0;
    bool stop = false;
    std::string error;
    std::vector<std::thread> readers;

    std::deque<Job> jobs;
    int64_t next_ticket = 0, done_tickets = 0;
    int64_t first_failed_ticket = -1;     // copies from this ticket on did not happen
    std::thread uploader;
    bool uploader_started = false;

    double read_s = 0, wait_s = 0;
    int64_t bytes_read = 0, n_reads = 0;

};

void set_failed(Ring& r, const std::string& msg) {
    if (r.error.empty()) r.error = msg;
    r.cv_ready.notify_all();
    r.cv_done.notify_all();
    r.cv_job.notify_all();
}

// read [off, off + len) of fd into dst, accepting end of file once `need` bytes have arrived
bool pread_all(int fd, uint8_t* dst, int64_t len, int64_t off, int64_t need, std::string& err) {
    int64_t done = 0;
    while (done < len) {
        const ssize_t r = pread(fd, dst + done, (size_t)(len - done), off + done);
        if (r < 0 && errno == EINTR) continue;
        if (r < 0) { err = std::string("read failed: ") + strerror(errno); return false; }
        if (r == 0) {
            if (done >= need) return true;
            err = "unexpected end of file";
            return false;
        }
        done += r;
    }
    return true;
}

// one piece into dst. O_DIRECT reads go through the reader's aligned scratch buffer in chunks of kChunk: the ring's
// page-locked buffers (hipHostMalloc) refuse direct I/O into them (EFAULT), and a block's range rarely starts at
// a 4 KiB boundary of the file anyway. Ordinary reads go straight to dst.
constexpr int64_t kChunk = int64_t(8) << 20;

bool read_piece(int fd, bool direct, const Piece& p, uint8_t* dst, uint8_t* scratch, std::string& err) {
    if (!direct) return pread_all(fd, dst, p.len, p.off, p.len, err);
    const int64_t end = p.off + p.len;
    for (int64_t cs = align_down(p.off); cs < end; cs += kChunk) {
        const int64_t ce = std::min(cs + kChunk, align_up(end));
        if (!pread_all(fd, scratch, ce - cs, cs, std::min(ce, end) - cs, err)) return false;
        const int64_t a = std::max(cs, p.off), b = std::min(ce, end);
        memcpy(dst + (a - p.off), scratch + (a - cs), (size_t)(b - a));
    }
    return true;
}

// one block into buffer `buf` (packed: piece k at its block offset); false with err set on failure
bool read_block(const Ring& r, int fd, bool direct, int64_t b, uint8_t* buf, uint8_t* scratch, std::string& err) {
    for (int64_t k = r.pstart[b]; k < r.pstart[b + 1]; k++) {
        const Piece& p = r.pieces[k];
        if (!read_piece(fd, direct, p, buf + p.dst, scratch, err)) return false;
    }
    return true;
}

void reader_main(Ring* rp) {
    Ring& r = *rp;
    if (r.pinned) (void)hipSetDevice(r.device);
    bool direct = r.direct;
    int fd = open(r.path.c_str(), O_RDONLY | O_CLOEXEC | (direct ? O_DIRECT : 0));
    if (fd < 0 && direct) {          // O_DIRECT refused (e.g. tmpfs): ordinary reads of the same ranges
        direct = false;
        fd = open(r.path.c_str(), O_RDONLY | O_CLOEXEC);
    }
    if (fd < 0) {
        std::lock_guard<std::mutex> g(r.m);
        set_failed(r, "open " + r.path + ": " + strerror(errno));
        return;
    }
    uint8_t* scratch = nullptr;
    if (direct) {
        scratch = static_cast<uint8_t*>(aligned_alloc(kAlign, (size_t)kChunk));
        if (!scratch) {
            std::lock_guard<std::mutex> g(r.m);
            set_failed(r, "scratch allocation failed");
            close(fd);
            return;
        }
    }
    for (;;) {
        int64_t pos;
        int s;
        hipEvent_t ev = nullptr;
        {
            std::unique_lock<std::mutex> lk(r.m);
            r.cv_read.wait(lk, [&] { return r.stop || !r.reads.empty(); });
            if (r.stop) break;
            pos = r.reads.front().first;
            s = r.reads.front().second;
            r.reads.pop_front();
            if (r.slots[s].copy_pending) {
                ev = r.slots[s].copy_ev;
                r.slots[s].copy_pending = false;
            }
        }
        if (ev) {
            const hipError_t e = hipEventSynchronize(ev);   // the previous copy out of this buffer has finished
            if (e != hipSuccess) {
                std::lock_guard<std::mutex> g(r.m);
                set_failed(r, std::string("hipEventSynchronize: ") + hipGetErrorString(e));
                continue;
            }
        }
        const int64_t b = pos % r.n_blocks;
        std::string err;
        const double t0 = now_s();
        const bool ok = read_block(r, fd, direct, b, r.bufs + (int64_t)s * r.buf_bytes, scratch, err);
        const double dt = now_s() - t0;
        std::lock_guard<std::mutex> g(r.m);
        if (!ok) {
            set_failed(r, "block " + std::to_string(b) + ": " + err);
            continue;
        }
        r.read_s += dt;
        r.bytes_read += r.block_bytes[b];
        r.n_reads++;
        Slot& sl = r.slots[s];
        sl.pos = pos;
        sl.nbytes = r.block_bytes[b];
        sl.ready = true;
        r.cv_ready.notify_all();
    }
    free(scratch);
    close(fd);
}

void request_next(Ring& r) {      // under r.m
    const int64_t pos = r.req++;
    const int s = (int)(pos % r.depth);
    r.slots[s].ready = false;
    r.reads.emplace_back(pos, s);
    r.cv_read.notify_one();
}

void prime(Ring& r) {             // under r.m
    while (r.req - r.cons < r.depth) request_next(r);
}

// wait for block `b` (the next in order) and return its buffer; under lk. A block already read is served even
// after a later read failed (the failure surfaces at the first block it kept from being read).
int acquire_locked(Ring& r, std::unique_lock<std::mutex>& lk, int64_t b, uint8_t** ptr, int64_t* nbytes, int* slot) {
    if (r.cons % r.n_blocks != b) {
        set_error("ssd ring out of sync: expected block %lld, got %lld", (long long)(r.cons % r.n_blocks), (long long)b);
        return WF_EINVAL;
    }
    const int s = (int)(r.cons % r.depth);
    auto have = [&] { return r.slots[s].ready && r.slots[s].pos == r.cons; };
    const double t0 = now_s();
    r.cv_ready.wait(lk, [&] { return r.stop || !r.error.empty() || have(); });
    r.wait_s += now_s() - t0;
    if (!have()) {
        if (r.error.empty()) set_error("ssd ring: closed while waiting for block %lld", (long long)b);
        else set_error("ssd ring: %s", r.error.c_str());
        return r.error.empty() ? WF_EINVAL : WF_EHIP;
    }
    *ptr = r.bufs + (int64_t)s * r.buf_bytes;
    *nbytes = r.slots[s].nbytes;
    *slot = s;
    return WF_OK;
}

void release_locked(Ring& r, int s) {
    r.slots[s].ready = false;
    r.cons++;
    request_next(r);
}

void uploader_main(Ring* rp) {
    Ring& r = *rp;
    (void)hipSetDevice(r.device);
    std::unique_lock<std::mutex> lk(r.m);
    for (;;) {
        r.cv_job.wait(lk, [&] { return r.stop || !r.jobs.empty(); });
        if (r.stop) return;
        Job j = r.jobs.front();
        r.jobs.pop_front();
        uint8_t* src;
        int64_t n;
        int s;
        if (acquire_locked(r, lk, j.block, &src, &n, &s) != WF_OK) {
            if (r.stop) return;
            set_failed(r, wf_last_error());
            if (r.first_failed_ticket < 0) r.first_failed_ticket = j.ticket;
            r.done_tickets = j.ticket + 1;
            r.cv_done.notify_all();
            continue;
        }
        lk.unlock();
        hipError_t e = hipSuccess;
        if (n > j.dst_bytes) e = hipErrorInvalidValue;
        if (e == hipSuccess && j.wait_ev) e = hipStreamWaitEvent(j.stream, j.wait_ev, 0);
        if (e == hipSuccess) e = hipMemcpyAsync(j.dst, src, (size_t)n, hipMemcpyHostToDevice, j.stream);
        if (e == hipSuccess && j.done_ev) e = hipEventRecord(j.done_ev, j.stream);
        if (e == hipSuccess) e = hipEventRecord(r.slots[s].copy_ev, j.stream);
        lk.lock();
        if (e != hipSuccess) {
            set_failed(r, std::string(n > j.dst_bytes ? "block larger than its slot" : hipGetErrorString(e)));
            if (r.first_failed_ticket < 0) r.first_failed_ticket = j.ticket;
        } else {
            r.slots[s].copy_pending = true;
        }
        release_locked(r, s);
        r.done_tickets = j.ticket + 1;
        r.cv_done.notify_all();
    }
}

void start(Ring& r) {
    r.stop = false;
    r.req = r.cons = 0;
    r.reads.clear();
    for (Slot& s : r.slots) { s.ready = false; s.pos = -1; }
    for (int t = 0; t < r.n_threads; t++) r.readers.emplace_back(reader_main, &r);
    std::lock_guard<std::mutex> g(r.m);
    prime(r);
}

void stop_all(Ring& r) {
    {
        std::lock_guard<std::mutex> g(r.m);
        r.stop = true;
        r.cv_read.notify_all();
        r.cv_job.notify_all();
        r.cv_ready.notify_all();
    }
    for (std::thread& t : r.readers) t.join();
    r.readers.clear();
    if (r.uploader_started) {
        r.uploader.join();
        r.uploader_started = false;
    }
}

Ring* as_ring(void* h) { return static_cast<Ring*>(h); }

}  // namespace
}  // namespace wf

using wf::set_error;

extern "C" int wf_ring_open(const char* path, int64_t n_blocks, const int64_t* piece_start, const int64_t* piece_off,
                            const int64_t* piece_len, const int64_t* piece_dst, int depth, int threads, int flags,
                            int device, void** ring) {
    using namespace wf;
    if (!path || !piece_start || !piece_off || !piece_len || !piece_dst || !ring) {
        set_error("wf_ring_open: null argument");
        return WF_EINVAL;
    }
    *ring = nullptr;
    if (n_blocks <= 0 || depth < 1 || depth > 64 || threads < 1 || threads > 16 || (flags & ~3) != 0) {
        set_error("wf_ring_open: n_blocks %lld, depth %d, threads %d, flags %d", (long long)n_blocks, depth, threads,
                  flags);
        return WF_EINVAL;
    }
    struct stat st;
    if (stat(path, &st) != 0 || !S_ISREG(st.st_mode)) {
        set_error("wf_ring_open: %s is not a readable regular file", path);
        return WF_EINVAL;
    }
    Ring* r = new Ring();
    r->path = path;
    r->device = device;
    r->pinned = (flags & WF_RING_PINNED) != 0;
    r->direct = (flags & WF_RING_DIRECT) != 0;
    r->n_blocks = n_blocks;
    r->depth = depth;
    r->n_threads = std::min(threads, depth);
    r->pstart.assign(piece_start, piece_start + n_blocks + 1);
    auto bad = [&](const char* why, int64_t b) {
        set_error("wf_ring_open: block %lld: %s", (long long)b, why);
        delete r;
        return WF_EINVAL;
    };
    if (r->pstart[0] != 0) return bad("piece list does not start at 0", 0);
    for (int64_t b = 0; b < n_blocks; b++) {
        const int64_t p0 = r->pstart[b], p1 = r->pstart[b + 1];
        if (p1 <= p0 || p1 - p0 > (1 << 20)) return bad("no pieces (or too many)", b);
        int64_t packed = 0;
        for (int64_t k = p0; k < p1; k++) {
            const Piece p{piece_off[k], piece_len[k], piece_dst[k]};
            if (p.off < 0 || p.len <= 0 || p.dst < 0 || p.off > st.st_size || p.len > st.st_size - p.off)
                return bad("piece outside the file", b);
            if (p.dst > (int64_t(1) << 40) || p.len > (int64_t(1) << 40)) return bad("piece too large", b);
            if (k > p0 && p.dst < r->pieces.back().dst + r->pieces.back().len) return bad("pieces overlap or are out of order", b);
            r->pieces.push_back(p);
            packed = std::max(packed, p.dst + p.len);
        }
        r->block_bytes.push_back(packed);
        r->buf_bytes = std::max(r->buf_bytes, packed);
    }
    r->buf_bytes = align_up(r->buf_bytes);
    r->slots.resize(depth);
    const size_t total = (size_t)r->buf_bytes * depth;
    if (r->pinned) {
        hipError_t e = hipSetDevice(device);
        if (e == hipSuccess) e = hipHostMalloc((void**)&r->bufs, total, hipHostMallocDefault);
        for (int s = 0; e == hipSuccess && s < depth; s++)
            e = hipEventCreateWithFlags(&r->slots[s].copy_ev, hipEventDisableTiming);
        if (e != hipSuccess) {
            set_error("wf_ring_open: %s", hipGetErrorString(e));
            for (Slot& s : r->slots) if (s.copy_ev) (void)hipEventDestroy(s.copy_ev);
            if (r->bufs) (void)hipHostFree(r->bufs);
            delete r;
            return WF_EHIP;
        }
    } else {
        r->bufs = static_cast<uint8_t*>(aligned_alloc(kAlign, total));
        if (!r->bufs) { set_error("wf_ring_open: host allocation of %zu bytes failed", total); delete r; return WF_EINVAL; }
    }
    start(*r);
    *ring = r;
    return WF_OK;
}

extern "C" int wf_ring_acquire(void* ring, int64_t block, void** ptr, int64_t* nbytes, int* slot) {
    using namespace wf;
    if (!ring || !ptr || !nbytes || !slot) { set_error("wf_ring_acquire: null argument"); return WF_EINVAL; }
    Ring& r = *as_ring(ring);
    std::unique_lock<std::mutex> lk(r.m);
    uint8_t* p;
    const int rc = acquire_locked(r, lk, block, &p, nbytes, slot);
    *ptr = rc == WF_OK ? p : nullptr;
    return rc;
}

extern "C" int wf_ring_release(void* ring, int slot, void* stream) {
    using namespace wf;
    if (!ring) { set_error("wf_ring_release: null ring"); return WF_EINVAL; }
    Ring& r = *as_ring(ring);
    if (slot < 0 || slot >= r.depth) { set_error("wf_ring_release: slot %d", slot); return WF_EINVAL; }
    hipError_t e = hipSuccess;
    if (stream && r.pinned) e = hipEventRecord(r.slots[slot].copy_ev, static_cast<hipStream_t>(stream));
    std::lock_guard<std::mutex> g(r.m);
    if (slot != (int)(r.cons % r.depth) || !r.slots[slot].ready) {
        set_error("wf_ring_release: slot %d is not the one acquired last", slot);
        return WF_EINVAL;
    }
    if (e != hipSuccess) {
        set_failed(r, hipGetErrorString(e));
        set_error("wf_ring_release: %s", hipGetErrorString(e));
        return WF_EHIP;
    }
    if (stream && r.pinned) r.slots[slot].copy_pending = true;
    release_locked(r, slot);
    return WF_OK;
}

extern "C" int wf_ring_submit(void* ring, int64_t block, void* dst, int64_t dst_bytes, void* wait_event,
                              void* done_event, void* stream, int64_t* ticket) {
    using namespace wf;
    if (!ring || !dst || !ticket) { set_error("wf_ring_submit: null argument"); return WF_EINVAL; }
    Ring& r = *as_ring(ring);
    if (!r.pinned) { set_error("wf_ring_submit: the ring was opened without WF_RING_PINNED"); return WF_EINVAL; }
    if (block < 0 || block >= r.n_blocks) { set_error("wf_ring_submit: block %lld", (long long)block); return WF_EINVAL; }
    std::lock_guard<std::mutex> g(r.m);
    if (!r.uploader_started) {
        r.uploader = std::thread(uploader_main, &r);
        r.uploader_started = true;
    }
    Job j{block, r.next_ticket++, dst, dst_bytes, static_cast<hipEvent_t>(wait_event),
          static_cast<hipEvent_t>(done_event), static_cast<hipStream_t>(stream)};
    r.jobs.push_back(j);
    r.cv_job.notify_one();
    *ticket = j.ticket;
    return WF_OK;
}

extern "C" int wf_ring_wait(void* ring, int64_t ticket) {
    using namespace wf;
    if (!ring) { set_error("wf_ring_wait: null ring"); return WF_EINVAL; }
    Ring& r = *as_ring(ring);
    std::unique_lock<std::mutex> lk(r.m);
    if (ticket < 0 || ticket >= r.next_ticket) { set_error("wf_ring_wait: ticket %lld was not issued", (long long)ticket); return WF_EINVAL; }
    const double t0 = now_s();
    r.cv_done.wait(lk, [&] { return r.done_tickets > ticket || r.stop; });
    r.wait_s += now_s() - t0;
    if (r.done_tickets <= ticket) { set_error("ssd ring: stopped before copy %lld was issued", (long long)ticket); return WF_EINVAL; }
    if (r.first_failed_ticket >= 0 && ticket >= r.first_failed_ticket) {
        set_error("ssd ring: %s", r.error.c_str());
        return WF_EHIP;
    }
    return WF_OK;
}

extern "C" int wf_ring_resync(void* ring) {
    using namespace wf;
    if (!ring) { set_error("wf_ring_resync: null ring"); return WF_EINVAL; }
    Ring& r = *as_ring(ring);
    {
        std::lock_guard<std::mutex> g(r.m);
        if (!r.jobs.empty() || r.done_tickets != r.next_ticket) {
            set_error("wf_ring_resync: submitted copies are still pending (wait for them first)");
            return WF_EINVAL;
        }
    }
    stop_all(r);
    for (wf::Slot& s : r.slots) {
        if (s.copy_pending) {
            const hipError_t e = hipEventSynchronize(s.copy_ev);
            if (e != hipSuccess) { set_error("wf_ring_resync: %s", hipGetErrorString(e)); return WF_EHIP; }
            s.copy_pending = false;
        }
    }
    r.error.clear();
    r.first_failed_ticket = -1;
    start(r);
    return WF_OK;
}

extern "C" int wf_ring_stats(void* ring, double* read_s, double* wait_s, int64_t* bytes, int64_t* reads) {
    using namespace wf;
    if (!ring) { set_error("wf_ring_stats: null ring"); return WF_EINVAL; }
    Ring& r = *as_ring(ring);
    std::lock_guard<std::mutex> g(r.m);
    if (read_s) *read_s = r.read_s;
    if (wait_s) *wait_s = r.wait_s;
    if (bytes) *bytes = r.bytes_read;
    if (reads) *reads = r.n_reads;
    return WF_OK;
}

extern "C" int wf_ring_close(void* ring) {
    using namespace wf;
    if (!ring) return WF_OK;
    Ring* r = as_ring(ring);
    stop_all(*r);
    int rc = WF_OK;
    for (wf::Slot& s : r->slots) {
        if (s.copy_ev) {
            if (s.copy_pending && hipEventSynchronize(s.copy_ev) != hipSuccess) rc = WF_EHIP;
            (void)hipEventDestroy(s.copy_ev);
        }
    }
    if (r->pinned) (void)hipHostFree(r->bufs);
    else free(r->bufs);
    delete r;
    return rc;
}
