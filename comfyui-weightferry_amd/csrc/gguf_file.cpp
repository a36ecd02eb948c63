// GGUF file reader: the on-disk side of the dequantisation path. Parses a GGUF (version 2 or 3) header -- the
// metadata key/value pairs and the tensor table -- and gives each tensor's GGML type, dimensions and absolute byte
// range in the file, so the SSD tier can read quantised blocks straight from the model file into pinned memory.
//
// Format (the published GGUF specification; the reference reads these files through ComfyUI-GGUF / gguf-py, which
// are not vendored): little-endian; "GGUF", u32 version, u64 tensor count, u64 key/value count; each key/value is
// a string key (u64 length + bytes), a u32 value type and the value (types 0-12: u8, i8, u16, i16, u32, i32, f32,
// bool, string, array = u32 element type + u64 count + elements, u64, i64, f64); each tensor info is a string
// name, u32 dimension count, that many u64 dimensions (innermost first), u32 GGML type and u64 offset relative to
// the data section. The data section starts at the first multiple of general.alignment (u32, default 32) after
// the tensor table; every tensor offset is a multiple of it.
//
// The file is untrusted input: every count, length, dimension, type and offset is checked against the file size
// before use, and a malformed file is an error (WF_EINVAL with a message), never a read past a buffer.
#include <errno.h>
#include <stdint.h>
#include <fcntl.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <vector>

#include "host_common.h"

namespace wf {
namespace {

// GGML block geometry: values per block and bytes per block (0 = type not handled)
struct TypeGeom { int64_t block, bytes; };
TypeGeom type_geom(uint32_t t) {
    switch (t) {
        case 0: return {1, 4};      // F32
        case 1: return {1, 2};      // F16
        case 2: return {32, 18};    // Q4_0
        case 3: return {32, 20};    // Q4_1
        case 6: return {32, 22};    // Q5_0
        case 7: return {32, 24};    // Q5_1
        case 8: return {32, 34};    // Q8_0
        case 10: return {256, 84};  // Q2_K
        case 11: return {256, 110}; // Q3_K
        case 12: return {256, 144}; // Q4_K
        case 13: return {256, 176}; // Q5_K
        case 14: return {256, 210}; // Q6_K
        case 30: return {1, 2};     // BF16
        default: return {0, 0};
    }
}

constexpr uint64_t kMaxCount = 1u << 24;       // tensors, key/values
constexpr uint64_t kMaxString = 1u << 26;      // bytes of one string

struct Tensor {
    std::string name;
    uint32_t type;
    uint32_t n_dims;
    int64_t dims[4];
    int64_t offset;       // absolute, in the file
    int64_t nbytes;
};

struct KV {
    std::string key;
    uint32_t type;        // value type; for arrays 9 with elem_type / count
    uint32_t elem_type = 0;
    uint64_t count = 0;
    int64_t i = 0;        // integer and bool values
    uint64_t u = 0;       // unsigned 64-bit values
    double f = 0;         // float values
    std::string s;        // string values
};

struct File {
    int fd = -1;
    int64_t size = 0;
    uint32_t version = 0;
    uint32_t alignment = 32;
    int64_t data_offset = 0;
    std::vector<KV> kvs;
    std::vector<Tensor> tensors;
};

// buffered sequential reader over pread with a hard end at the file size
class Cursor {
  public:
    Cursor(int fd, int64_t size) : fd_(fd), size_(size) {}
    int64_t pos() const { return pos_; }
    bool bytes(void* dst, uint64_t n) {
        if (n > (uint64_t)(size_ - pos_)) return fail("truncated file");
        uint8_t* d = static_cast<uint8_t*>(dst);
        while (n) {
            if (bpos_ >= blen_) {
                if (!fill()) return false;
            }
            const uint64_t k = std::min<uint64_t>(n, blen_ - bpos_);
            memcpy(d, buf_ + bpos_, k);
            d += k;
            bpos_ += k;
            pos_ += k;
            n -= k;
        }
        return true;
    }
    bool skip(uint64_t n) {
        if (n > (uint64_t)(size_ - pos_)) return fail("truncated file");
        const uint64_t in_buf = blen_ - bpos_;
        if (n <= in_buf) {
            bpos_ += n;
        } else {
            bpos_ = blen_ = 0;
            base_ = pos_ + n;
        }
        pos_ += n;
        return true;
    }
    template <typename T>
    bool pod(T& v) { return bytes(&v, sizeof(T)); }
    bool str(std::string& s) {
        uint64_t n;
        if (!pod(n)) return false;
        if (n > kMaxString) return fail("string length beyond the reader's limit");
        s.resize(n);
        return n == 0 || bytes(&s[0], n);
    }
    bool fail(const char* why) {
        if (!err_) set_error("gguf: %s at byte %lld", why, (long long)pos_);
        err_ = true;
        return false;
    }
    bool failed() const { return err_; }

  private:
    bool fill() {
        base_ = pos_;
        const int64_t want = std::min<int64_t>(sizeof(buf_), size_ - pos_);
        int64_t got = 0;
        while (got < want) {
            const ssize_t r = pread(fd_, buf_ + got, want - got, base_ + got);
            if (r < 0 && errno == EINTR) continue;
            if (r <= 0) return fail(r < 0 ? strerror(errno) : "unexpected end of file");
            got += r;
        }
        bpos_ = 0;
        blen_ = got;
        return true;
    }
    int fd_;
    int64_t size_;
    int64_t pos_ = 0, base_ = 0;
    uint8_t buf_[1 << 16];
    uint64_t bpos_ = 0, blen_ = 0;
    bool err_ = false;
};

bool scalar_size(uint32_t t, uint64_t& n) {
    static const uint64_t sz[] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
    if (t > 12 || t == 8 || t == 9) return false;
    n = sz[t];
    return true;
}

bool read_scalar(Cursor& c, uint32_t t, KV& kv) {
    switch (t) {
        case 0: { uint8_t v; if (!c.pod(v)) return false; kv.i = v; kv.u = v; kv.f = v; return true; }
        case 1: { int8_t v; if (!c.pod(v)) return false; kv.i = v; kv.f = v; return true; }
        case 2: { uint16_t v; if (!c.pod(v)) return false; kv.i = v; kv.u = v; kv.f = v; return true; }
        case 3: { int16_t v; if (!c.pod(v)) return false; kv.i = v; kv.f = v; return true; }
        case 4: { uint32_t v; if (!c.pod(v)) return false; kv.i = v; kv.u = v; kv.f = v; return true; }
        case 5: { int32_t v; if (!c.pod(v)) return false; kv.i = v; kv.f = v; return true; }
        case 6: { float v; if (!c.pod(v)) return false; kv.f = v; return true; }
        case 7: {
            uint8_t v;
            if (!c.pod(v)) return false;
            if (v > 1) return c.fail("bool value other than 0 or 1");
            kv.i = v;
            return true;
        }
        case 10: { uint64_t v; if (!c.pod(v)) return false; kv.u = v; kv.i = (int64_t)v; kv.f = (double)v; return true; }
        case 11: { int64_t v; if (!c.pod(v)) return false; kv.i = v; kv.f = (double)v; return true; }
        case 12: { double v; if (!c.pod(v)) return false; kv.f = v; return true; }
        default: return c.fail("unknown value type");
    }
}

bool parse(File& f) {
    Cursor c(f.fd, f.size);
    char magic[4];
    if (!c.bytes(magic, 4)) return false;
    if (memcmp(magic, "GGUF", 4) != 0) return c.fail("not a GGUF file (magic)");
    if (!c.pod(f.version)) return false;
    if (f.version != 2 && f.version != 3) return c.fail("GGUF version other than 2 or 3");
    uint64_t n_tensors, n_kv;
    if (!c.pod(n_tensors) || !c.pod(n_kv)) return false;
    if (n_tensors > kMaxCount || n_kv > kMaxCount) return c.fail("tensor or key/value count beyond the reader's limit");
    f.kvs.reserve(n_kv);
    for (uint64_t i = 0; i < n_kv; i++) {
        KV kv;
        if (!c.str(kv.key) || !c.pod(kv.type)) return false;
        if (kv.type == 8) {
            if (!c.str(kv.s)) return false;
        } else if (kv.type == 9) {
            if (!c.pod(kv.elem_type) || !c.pod(kv.count)) return false;
            if (kv.elem_type == 9) return c.fail("nested arrays are not handled");
            if (kv.elem_type == 8) {
                for (uint64_t k = 0; k < kv.count; k++) {
                    uint64_t n;
                    if (!c.pod(n)) return false;
                    if (!c.skip(n)) return false;
                }
            } else {
                uint64_t es;
                if (!scalar_size(kv.elem_type, es)) return c.fail("unknown array element type");
                if (kv.count > (uint64_t)f.size / es) return c.fail("array longer than the file");
                if (!c.skip(kv.count * es)) return false;
            }
        } else if (!read_scalar(c, kv.type, kv)) {
            return false;
        }
        if (kv.key == "general.alignment") {
            if (kv.type != 4 || kv.u == 0 || (kv.u & (kv.u - 1)) != 0 || kv.u > (1u << 20))
                return c.fail("general.alignment must be a power-of-two u32");
            f.alignment = (uint32_t)kv.u;
        }
        f.kvs.push_back(std::move(kv));
    }
    f.tensors.reserve(n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
        Tensor t;
        if (!c.str(t.name) || !c.pod(t.n_dims)) return false;
        if (t.n_dims < 1 || t.n_dims > 4) return c.fail("tensor with a dimension count other than 1-4");
        int64_t elems = 1;
        for (uint32_t d = 0; d < 4; d++) t.dims[d] = 1;
        for (uint32_t d = 0; d < t.n_dims; d++) {
            uint64_t v;
            if (!c.pod(v)) return false;
            if (v == 0 || v > (1ull << 40)) return c.fail("tensor dimension of 0 or beyond 2^40");
            t.dims[d] = (int64_t)v;
            if (elems > (int64_t)((1ull << 62) / v)) return c.fail("tensor element count overflows");
            elems *= (int64_t)v;
        }
        uint64_t off;
        if (!c.pod(t.type) || !c.pod(off)) return false;
        const TypeGeom g = type_geom(t.type);
        if (g.block == 0) return c.fail("tensor of a GGML type this reader does not size");
        if (t.dims[0] % g.block != 0) return c.fail("row length not a whole number of blocks");
        const int64_t blocks = elems / g.block;
        if (blocks > INT64_MAX / g.bytes) return c.fail("tensor byte count overflows");
        t.nbytes = blocks * g.bytes;
        if (t.nbytes <= 0) return c.fail("tensor of no bytes");
        if (off > (uint64_t)f.size) return c.fail("tensor offset beyond the file");
        t.offset = (int64_t)off;     // relative until the data section is known
        f.tensors.push_back(std::move(t));
    }
    const int64_t a = f.alignment;
    f.data_offset = (c.pos() + a - 1) / a * a;
    for (Tensor& t : f.tensors) {
        if (t.offset % a != 0) {
            set_error("gguf: tensor %s offset %lld is not a multiple of the alignment %lld", t.name.c_str(),
                      (long long)t.offset, (long long)a);
            return false;
        }
        t.offset += f.data_offset;
        if (t.offset > f.size || t.nbytes > f.size - t.offset) {
            set_error("gguf: tensor %s [%lld, +%lld) lies beyond the file's %lld bytes", t.name.c_str(),
                      (long long)t.offset, (long long)t.nbytes, (long long)f.size);
            return false;
        }
    }
    return true;
}

File* as_file(void* h) { return static_cast<File*>(h); }

}  // namespace
}  // namespace wf

using wf::set_error;

extern "C" int wf_gguf_open(const char* path, void** handle) {
    if (!path || !handle) { set_error("wf_gguf_open: null argument"); return WF_EINVAL; }
    *handle = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) { set_error("wf_gguf_open: %s: %s", path, strerror(errno)); return WF_EINVAL; }
    struct stat st;
    if (fstat(fd, &st) != 0 || !S_ISREG(st.st_mode)) {
        set_error("wf_gguf_open: %s is not a regular file", path);
        close(fd);
        return WF_EINVAL;
    }
    wf::File* f = new wf::File();
    f->fd = fd;
    f->size = st.st_size;
    const bool ok = wf::parse(*f);
    close(fd);
    f->fd = -1;
    if (!ok) {
        delete f;
        return WF_EINVAL;
    }
    *handle = f;
    return WF_OK;
}

extern "C" int wf_gguf_close(void* handle) {
    delete wf::as_file(handle);
    return WF_OK;
}

extern "C" int wf_gguf_info(void* handle, int* version, int64_t* n_tensors, int64_t* n_kv, int64_t* alignment,
                            int64_t* data_offset, int64_t* file_bytes) {
    if (!handle) { set_error("wf_gguf_info: null handle"); return WF_EINVAL; }
    const wf::File* f = wf::as_file(handle);
    if (version) *version = (int)f->version;
    if (n_tensors) *n_tensors = (int64_t)f->tensors.size();
    if (n_kv) *n_kv = (int64_t)f->kvs.size();
    if (alignment) *alignment = f->alignment;
    if (data_offset) *data_offset = f->data_offset;
    if (file_bytes) *file_bytes = f->size;
    return WF_OK;
}

static int copy_name(const std::string& s, char* buf, int64_t cap) {
    if (!buf || cap <= 0) return (int)s.size();
    const int64_t n = std::min<int64_t>((int64_t)s.size(), cap - 1);
    memcpy(buf, s.data(), n);
    buf[n] = 0;
    return (int)s.size();
}

extern "C" int wf_gguf_tensor(void* handle, int64_t i, char* name, int64_t name_cap, int* type, int* n_dims,
                              int64_t* dims4, int64_t* offset, int64_t* nbytes) {
    if (!handle) { set_error("wf_gguf_tensor: null handle"); return WF_EINVAL; }
    const wf::File* f = wf::as_file(handle);
    if (i < 0 || i >= (int64_t)f->tensors.size()) { set_error("wf_gguf_tensor: index %lld", (long long)i); return WF_EINVAL; }
    const wf::Tensor& t = f->tensors[i];
    if (name && name_cap > 0 && (int64_t)t.name.size() >= name_cap) {
        set_error("wf_gguf_tensor: name of %zu bytes does not fit %lld", t.name.size(), (long long)name_cap);
        return WF_EINVAL;
    }
    copy_name(t.name, name, name_cap);
    if (type) *type = (int)t.type;
    if (n_dims) *n_dims = (int)t.n_dims;
    if (dims4) for (int d = 0; d < 4; d++) dims4[d] = t.dims[d];
    if (offset) *offset = t.offset;
    if (nbytes) *nbytes = t.nbytes;
    return WF_OK;
}

extern "C" int wf_gguf_kv(void* handle, int64_t i, char* key, int64_t key_cap, int* type, int* elem_type,
                          int64_t* count, int64_t* ival, double* fval, char* sval, int64_t sval_cap) {
    if (!handle) { set_error("wf_gguf_kv: null handle"); return WF_EINVAL; }
    const wf::File* f = wf::as_file(handle);
    if (i < 0 || i >= (int64_t)f->kvs.size()) { set_error("wf_gguf_kv: index %lld", (long long)i); return WF_EINVAL; }
    const wf::KV& kv = f->kvs[i];
    if (key && key_cap > 0 && (int64_t)kv.key.size() >= key_cap) {
        set_error("wf_gguf_kv: key of %zu bytes does not fit %lld", kv.key.size(), (long long)key_cap);
        return WF_EINVAL;
    }
    if (kv.type == 8 && sval && sval_cap > 0 && (int64_t)kv.s.size() >= sval_cap) {
        set_error("wf_gguf_kv: string value of %zu bytes does not fit %lld", kv.s.size(), (long long)sval_cap);
        return WF_EINVAL;
    }
    copy_name(kv.key, key, key_cap);
    if (type) *type = (int)kv.type;
    if (elem_type) *elem_type = (int)kv.elem_type;
    if (count) *count = (int64_t)(kv.type == 8 ? kv.s.size() : kv.count);
    if (ival) *ival = kv.type == 10 ? (int64_t)kv.u : kv.i;
    if (fval) *fval = kv.f;
    if (kv.type == 8) copy_name(kv.s, sval, sval_cap);
    return WF_OK;
}
