// wfp_hbm_stream: a measuring kernel, built into its own library (libwf_probe.so) for the benchmark and never
// linked into libweightferry_hip.so. It moves the same bytes as a dequantisation launch with no arithmetic -- each
// thread reads R 16-byte chunks and writes W (non-temporal, as the dequantisation kernels store) -- so the benchmark
// can set a kernel's rate beside what HBM delivers for the same read:write mix and size.
//
// int wfp_hbm_stream(const void* in, void* out, int64_t items, int reads, int writes, void* stream): thread t reads
// in[t + r * items] (r < reads) and writes out[t + w * items] (w < writes); mixes 1:0, 0:1, 1:1, 1:2, 2:7; `out` is
// required (16 bytes at least for the read-only mix, which may store one word there). 0 on success, -1 for bad
// arguments, -2 for an unsupported mix, -3 for a launch error; wfp_last_error() gives the message.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

namespace {
thread_local char g_err[256] = "";

void fail(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
}  // namespace

namespace wfp {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

template <int R, int W>
__global__ __launch_bounds__(256) void hbm_stream(const uint4* __restrict__ in, uint4* __restrict__ out, int64_t items,
                                                  unsigned key, unsigned* __restrict__ sink) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= items) return;
    unsigned acc = 0;
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint4 v = in[t + r * items];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
#pragma unroll
    for (int w = 0; w < W; w++) {
        const u32x4 v = {acc, (unsigned)w, (unsigned)t, 0u};
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(out + t + w * items));
    }
    // the read-only form keeps its loads: the sum goes to the sink when it equals a key the compiler cannot see
    if (W == 0 && acc == key) sink[0] = acc;
}

template <int R, int W>
static void launch_stream(const void* in, void* out, int64_t items, hipStream_t s) {
    const int64_t grid = (items + 255) / 256;
    hbm_stream<R, W><<<dim3((unsigned)grid), 256, 0, s>>>(static_cast<const uint4*>(in), static_cast<uint4*>(out),
                                                          items, 0x9e3779b9u, static_cast<unsigned*>(out));
}

}  // namespace wfp

extern "C" const char* wfp_last_error(void) { return g_err; }

extern "C" int wfp_hbm_stream(const void* in, void* out, int64_t items, int reads, int writes, void* stream) {
    using namespace wfp;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (items <= 0 || items > ((int64_t)1 << 31) * 255) {
        fail("wfp_hbm_stream: %lld items", (long long)items);
        return -1;
    }
    if ((reads > 0 && !in) || !out || !aligned16(in) || !aligned16(out)) {
        fail("wfp_hbm_stream: null or misaligned buffer");
        return -1;
    }
    if (reads == 1 && writes == 0) launch_stream<1, 0>(in, out, items, s);
    else if (reads == 0 && writes == 1) launch_stream<0, 1>(in, out, items, s);
    else if (reads == 1 && writes == 1) launch_stream<1, 1>(in, out, items, s);
    else if (reads == 1 && writes == 2) launch_stream<1, 2>(in, out, items, s);
    else if (reads == 2 && writes == 7) launch_stream<2, 7>(in, out, items, s);
    else {
        fail("wfp_hbm_stream: mix %d:%d (supported 1:0, 0:1, 1:1, 1:2, 2:7)", reads, writes);
        return -2;
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        fail("wfp_hbm_stream launch: %s", hipGetErrorString(e));
        return -3;
    }
    return 0;
}
