// The C ABI of include/bchip.h: context, device memory, argument checks and dispatch.
//
// It stands where bc-infer's CUDA backend stands (crates/bc-infer/src/gpu/cuda.rs:1-95):
// one device, one stream, launches queued back to back and waited for by bchip_sync. Each
// entry point checks its arguments on the host before anything reaches the GPU: shapes the
// kernels assume, alignment, and, for buffers this library allocated, that every byte a
// kernel will touch lies inside them. Errors come back as codes with a thread-local
// message; nothing aborts across the ABI.
#include "bchip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "common.hpp"
#include "internal.hpp"

using namespace bchip;

// The scratch of bchip_rope_append_attention_noalloc: a one-row step's chunk states
// (NOALLOC_O_BYTES: 1024 units x 16 slots x 256 dims, the most a one-row plan takes for
// nkv <= 1024), their maxima and sums, and a fused step's staged rotated q (nh * hd <= 65536).
// Each device holds its own copy from the library's load until the process ends; every call
// on one device shares it, so calls on one device that overlap in time race. Host code never
// names it: bchip_init takes its device address (hipGetSymbolAddress) and uses that.
constexpr size_t NOALLOC_O_BYTES = (size_t)16 << 20;
constexpr size_t NOALLOC_ML_BYTES = (size_t)128 << 10;
constexpr size_t NOALLOC_Q_BYTES = (size_t)256 << 10;
constexpr size_t NOALLOC_BYTES = NOALLOC_O_BYTES + NOALLOC_ML_BYTES + NOALLOC_Q_BYTES;
static __device__ __align__(256) unsigned char scratch[NOALLOC_BYTES];

struct bchip_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t t0 = nullptr, t1 = nullptr;
    Workspace ws;
    Workspace fixed_ws;  // the scratch array's device copy, for the no-allocation entry point
    uint32_t* mm_cnt = nullptr;  // the batched products' arrival counters (MATMUL_COUNTERS, zero between calls)
    std::map<uintptr_t, size_t> allocs;  // base -> bytes, of bchip_alloc memory
    std::string name;
    hipEvent_t arm_before = nullptr, arm_after = nullptr;  // bchip_timer_arm, for the next call
    // The armed events, handed to one attention call and cleared.
    void take_marks(bchip::AttnCall& a) {
        a.ev_before = arm_before;
        a.ev_after = arm_after;
        arm_before = arm_after = nullptr;
    }
    // Hands an arming taken by a call that launched nothing back for the call after it.
    void restore_marks(const bchip::AttnCall& a) {
        arm_before = a.ev_before;
        arm_after = a.ev_after;
    }
};

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    if (e == hipErrorOutOfMemory) return fail(BCHIP_E_OOM, "%s: %s", what, hipGetErrorString(e));
    return fail(BCHIP_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define HIP_TRY(expr, what)                       \
    do {                                          \
        hipError_t e_ = (expr);                   \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

int enter(bchip_ctx* c) {
    if (!c) return fail(BCHIP_E_ARG, "no context");
    hipError_t e = hipSetDevice(c->device);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    return BCHIP_OK;
}

// After the stream has drained: a single-launch fold whose wait for the other workgroups of
// its group ran out (other work held the CUs they needed) wrote NaN for its outputs and set
// the error word. Reported once, then cleared.
int fold_status(bchip_ctx* c) {
    if (c->ws.gerr_host && *c->ws.gerr_host) {
        *c->ws.gerr_host = 0;
        // The stream has drained: no fold is waiting, so the counters can start over.
        (void)hipMemset(c->ws.gcnt, 0, (size_t)GROUP_COUNTERS * GROUP_STRIDE * sizeof(uint32_t));
        return fail(BCHIP_E_HIP, "an attention fold timed out waiting for its workgroups (other kernels held "
                                 "the GPU); that call's outputs are NaN");
    }
    return BCHIP_OK;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Byte counts from element counts, saturated: a count that overflows 64 bits becomes
// UINT64_MAX, which no span check accepts.
uint64_t sat_add(uint64_t a, uint64_t b) {
    uint64_t r;
    return __builtin_add_overflow(a, b, &r) ? UINT64_MAX : r;
}
uint64_t sat_mul(uint64_t a, uint64_t b) {
    uint64_t r;
    return __builtin_mul_overflow(a, b, &r) ? UINT64_MAX : r;
}

// [p + off, p + off + bytes) must not wrap the address space (whoever allocated p), and,
// when p lies in memory this library allocated, must lie inside that allocation. Memory
// from elsewhere cannot be checked further and is trusted.
int check_at(const bchip_ctx* c, const void* p, uint64_t off, uint64_t bytes, const char* what) {
    if (bytes == 0) return BCHIP_OK;
    const uintptr_t a = (uintptr_t)p;
    if (off == UINT64_MAX || bytes == UINT64_MAX || off > UINTPTR_MAX - a || bytes > UINTPTR_MAX - a - off)
        return fail(BCHIP_E_ARG, "%s: a span of %llu bytes at offset %llu passes the end of the address space", what,
                    (unsigned long long)bytes, (unsigned long long)off);
    if (c->allocs.empty()) return BCHIP_OK;
    auto it = c->allocs.upper_bound(a);
    if (it == c->allocs.begin()) return BCHIP_OK;
    --it;
    if (a >= it->first + it->second) return BCHIP_OK;  // not ours
    const uint64_t left = it->first + it->second - a;  // bytes from p to the allocation's end
    if (off > left || bytes > left - off)
        return fail(BCHIP_E_ARG, "%s: %llu bytes from offset %llu pass the end of its %llu-byte buffer", what,
                    (unsigned long long)bytes, (unsigned long long)(a - it->first + off),
                    (unsigned long long)it->second);
    return BCHIP_OK;
}

int check_span(const bchip_ctx* c, const void* p, uint64_t bytes, const char* what) {
    return check_at(c, p, 0, bytes, what);
}

uint32_t esize(uint32_t type) { return type == BCHIP_F16 ? 2u : 4u; }

// Bytes from p to the end of the bchip_alloc allocation holding it, or UINT64_MAX for
// memory this library did not allocate.
uint64_t bytes_left(const bchip_ctx* c, const void* p) {
    const uintptr_t a = (uintptr_t)p;
    auto it = c->allocs.upper_bound(a);
    if (it == c->allocs.begin()) return UINT64_MAX;
    --it;
    if (a >= it->first + it->second) return UINT64_MAX;
    return it->first + it->second - a;
}

#define CHECK(expr)                  \
    do {                             \
        int rc_ = (expr);            \
        if (rc_ != BCHIP_OK) return rc_; \
    } while (0)

int check_heads(uint32_t nh, uint32_t nkv, uint32_t hd) {
    if (nh == 0 || nkv == 0 || nh % nkv != 0)
        return fail(BCHIP_E_UNSUPPORTED, "%u query heads do not share %u KV heads evenly", nh, nkv);
    if (nh / nkv > 16) return fail(BCHIP_E_UNSUPPORTED, "group of %u query heads per KV head (at most 16)", nh / nkv);
    if (hd == 0 || hd % 8 != 0 || hd > MAX_HD)
        return fail(BCHIP_E_UNSUPPORTED, "head_dim %u (a multiple of 8 up to %u)", hd, MAX_HD);
    return BCHIP_OK;
}

}  // namespace

namespace bchip {

void Workspace::set_fixed(void* base, size_t o_bytes, size_t ml_bytes, size_t q_bytes, const Workspace& owner) {
    fixed = true;
    o = (float*)base;
    ml = (float*)((char*)base + o_bytes);
    qrot = (float*)((char*)base + o_bytes + ml_bytes);
    o_cap = o_bytes;
    ml_cap = ml_bytes;
    qrot_cap = q_bytes;
    zero = owner.zero;
    gcnt = owner.gcnt;
    cus = owner.cus;
    group_fold = owner.group_fold;
    group_spread = owner.group_spread;
    group_spins = owner.group_spins;
    combine_long = owner.combine_long;
    row_runs = owner.row_runs;
    gerr = owner.gerr;
    gerr_host = owner.gerr_host;
}

hipError_t Workspace::reserve(size_t need_slots, size_t hd_pad) {
    if (fixed) {
        if (need_slots * hd_pad * sizeof(float) > o_cap || need_slots * 2 * sizeof(float) > ml_cap)
            return hipErrorOutOfMemory;
        slots = need_slots;
        hdp = hd_pad;
        return hipSuccess;
    }
    if (need_slots <= slots && hd_pad <= hdp && o) return hipSuccess;
    const size_t ns = std::max(need_slots, slots), nh = std::max(hd_pad, hdp);
    if (o) (void)hipFree(o);
    if (ml) (void)hipFree(ml);
    o = ml = nullptr;
    slots = 0;
    hdp = nh;
    hipError_t e = hipMalloc((void**)&o, ns * hdp * sizeof(float));
    if (e != hipSuccess) return e;
    e = hipMalloc((void**)&ml, ns * 2 * sizeof(float));
    if (e != hipSuccess) return e;
    slots = ns;
    return hipSuccess;
}

hipError_t Workspace::reserve_vt(size_t bytes) {
    if (fixed) return hipErrorOutOfMemory;
    if (bytes <= vt_bytes && vt) return hipSuccess;
    if (vt) (void)hipFree(vt);
    vt = nullptr;
    vt_bytes = 0;
    hipError_t e = hipMalloc(&vt, bytes);
    if (e != hipSuccess) return e;
    vt_bytes = bytes;
    return hipSuccess;
}

hipError_t Workspace::reserve_qrot(size_t floats) {
    if (fixed) {
        if (floats * sizeof(float) > qrot_cap) return hipErrorOutOfMemory;
        qrot_floats = floats;
        return hipSuccess;
    }
    if (floats <= qrot_floats && qrot) return hipSuccess;
    if (qrot) (void)hipFree(qrot);
    qrot = nullptr;
    qrot_floats = 0;
    hipError_t e = hipMalloc((void**)&qrot, floats * sizeof(float));
    if (e != hipSuccess) return e;
    qrot_floats = floats;
    return hipSuccess;
}

hipError_t Workspace::init(int device) {
    hipError_t e = hipMalloc(&zero, ZERO_BYTES);
    if (e == hipSuccess) e = hipMemset(zero, 0, ZERO_BYTES);
    if (e == hipSuccess) e = hipMalloc((void**)&gcnt, (size_t)GROUP_COUNTERS * GROUP_STRIDE * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemset(gcnt, 0, (size_t)GROUP_COUNTERS * GROUP_STRIDE * sizeof(uint32_t));
    int n = 0;
    if (e == hipSuccess) e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device);
    cus = n > 0 ? (uint32_t)n : 0u;
    // A caller whose GPU runs other kernels beside this library's can turn the single-launch
    // folds off (their workgroups wait for each other; see attention.hip).
    const char* gf = getenv("BCHIP_GROUP_FOLD");
    group_fold = !(gf && strcmp(gf, "0") == 0);
    group_spread = gf && strcmp(gf, "spread") == 0;
    const char* cl = getenv("BCHIP_COMBINE_LONG");
    combine_long = !(cl && strcmp(cl, "0") == 0);
    if (const char* rr = getenv("BCHIP_ROW_RUNS")) row_runs = strcmp(rr, "0") == 0 ? 0u : strcmp(rr, "2") == 0 ? 2u : 1u;
    if (const char* sp = getenv("BCHIP_GROUP_FOLD_SPINS")) {
        const long v = strtol(sp, nullptr, 10);
        if (v > 0 && v < (1l << 24)) group_spins = (uint32_t)v;
    }
    void* h = nullptr;
    if (e == hipSuccess) e = hipHostMalloc(&h, 64, hipHostMallocMapped);
    if (e == hipSuccess) {
        gerr_host = (volatile uint32_t*)h;
        *gerr_host = 0;
        e = hipHostGetDevicePointer((void**)&gerr, h, 0);
    }
    return e;
}

void Workspace::release() {
    if (fixed) return;  // a view of memory this workspace does not own
    if (o) (void)hipFree(o);
    if (ml) (void)hipFree(ml);
    if (vt) (void)hipFree(vt);
    if (qrot) (void)hipFree(qrot);
    o = ml = nullptr;
    vt = nullptr;
    qrot = nullptr;
    qrot_floats = 0;
    vt_bytes = 0;
    slots = hdp = 0;
}

}  // namespace bchip

extern "C" {

const char* bchip_last_error(void) { return g_err.c_str(); }

int bchip_abi_version(void) { return BCHIP_ABI_VERSION; }

int bchip_init(int device, bchip_ctx** out) {
    if (!out) return fail(BCHIP_E_ARG, "no output pointer");
    *out = nullptr;
    const char* env = getenv("BC_INFER_GPU");
    if (env && strcmp(env, "0") == 0) return fail(BCHIP_E_DISABLED, "BC_INFER_GPU=0 turns the GPU off");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail(BCHIP_E_NODEV, "no HIP device");
    if (device < 0 || device >= n) return fail(BCHIP_E_NODEV, "device %d of %d", device, n);
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(BCHIP_E_NODEV, "device %d is %s; these kernels are built for gfx950", device, prop.gcnArchName);
    HIP_TRY(hipSetDevice(device), "hipSetDevice");
    bchip_ctx* c = new bchip_ctx();
    c->device = device;
    // The marketing name can be empty (some runtimes leave it blank): fall back to the ISA.
    c->name = std::string(prop.name[0] ? prop.name : prop.gcnArchName) + " (" +
              std::to_string(prop.multiProcessorCount) + " CUs)";
    hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = c->ws.init(device);
    if (e == hipSuccess) {
        // This device's copy of the no-allocation scratch (the device is current here).
        void* sp = nullptr;
        e = hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch));
        if (e == hipSuccess) c->fixed_ws.set_fixed(sp, NOALLOC_O_BYTES, NOALLOC_ML_BYTES, NOALLOC_Q_BYTES, c->ws);
    }
    if (e == hipSuccess) e = hipMalloc((void**)&c->mm_cnt, MATMUL_COUNTERS * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemset(c->mm_cnt, 0, MATMUL_COUNTERS * sizeof(uint32_t));
    if (e == hipSuccess) e = hipEventCreate(&c->t0);
    if (e == hipSuccess) e = hipEventCreate(&c->t1);
    if (e != hipSuccess) {
        bchip_destroy(c);
        return hip_fail(e, "creating the stream");
    }
    *out = c;
    return BCHIP_OK;
}

int bchip_destroy(bchip_ctx* c) {
    if (!c) return BCHIP_OK;
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    c->ws.release();
    if (c->ws.zero) (void)hipFree(c->ws.zero);
    if (c->ws.gcnt) (void)hipFree(c->ws.gcnt);
    if (c->ws.gerr_host) (void)hipHostFree((void*)c->ws.gerr_host);
    if (c->mm_cnt) (void)hipFree(c->mm_cnt);
    for (auto& a : c->allocs) (void)hipFree((void*)a.first);
    if (c->t0) (void)hipEventDestroy(c->t0);
    if (c->t1) (void)hipEventDestroy(c->t1);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
    return BCHIP_OK;
}

int bchip_device_name(bchip_ctx* c, char* buf, size_t len) {
    CHECK(enter(c));
    if (!buf || len == 0) return fail(BCHIP_E_ARG, "no buffer");
    snprintf(buf, len, "%s", c->name.c_str());
    return BCHIP_OK;
}

int bchip_mem_free(bchip_ctx* c, uint64_t* free_bytes) {
    CHECK(enter(c));
    if (!free_bytes) return fail(BCHIP_E_ARG, "no output pointer");
    size_t f = 0, t = 0;
    HIP_TRY(hipMemGetInfo(&f, &t), "hipMemGetInfo");
    *free_bytes = f;
    return BCHIP_OK;
}

int bchip_unified(bchip_ctx* c, int* unified) {
    CHECK(enter(c));
    if (!unified) return fail(BCHIP_E_ARG, "no output pointer");
    *unified = 0;
    return BCHIP_OK;
}

int bchip_alloc(bchip_ctx* c, size_t bytes, void** dev) {
    CHECK(enter(c));
    if (!dev) return fail(BCHIP_E_ARG, "no output pointer");
    *dev = nullptr;
    if (bytes == 0) bytes = 1;
    void* p = nullptr;
    HIP_TRY(hipMalloc(&p, bytes), "hipMalloc");
    hipError_t e = hipMemsetAsync(p, 0, bytes, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        (void)hipFree(p);
        return hip_fail(e, "zeroing a new buffer");
    }
    c->allocs[(uintptr_t)p] = bytes;
    *dev = p;
    return BCHIP_OK;
}

int bchip_free(bchip_ctx* c, void* dev) {
    CHECK(enter(c));
    if (!dev) return BCHIP_OK;
    auto it = c->allocs.find((uintptr_t)dev);
    if (it == c->allocs.end()) return fail(BCHIP_E_ARG, "%p was not allocated by this context", dev);
    HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    HIP_TRY(hipFree(dev), "hipFree");
    c->allocs.erase(it);
    return BCHIP_OK;
}

int bchip_upload(bchip_ctx* c, void* dev, size_t off, const void* host, size_t bytes) {
    CHECK(enter(c));
    if (bytes == 0) return BCHIP_OK;
    if (!dev || !host) return fail(BCHIP_E_ARG, "null pointer");
    CHECK(check_at(c, dev, off, bytes, "upload"));
    HIP_TRY(hipMemcpyAsync((char*)dev + off, host, bytes, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync");
    HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return BCHIP_OK;
}

int bchip_download(bchip_ctx* c, const void* dev, size_t off, void* host, size_t bytes) {
    CHECK(enter(c));
    if (bytes == 0) return BCHIP_OK;
    if (!dev || !host) return fail(BCHIP_E_ARG, "null pointer");
    CHECK(check_at(c, dev, off, bytes, "download"));
    HIP_TRY(hipMemcpyAsync(host, (const char*)dev + off, bytes, hipMemcpyDeviceToHost, c->stream), "hipMemcpyAsync");
    HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return fold_status(c);
}

int bchip_sync(bchip_ctx* c) {
    CHECK(enter(c));
    HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return fold_status(c);
}

int bchip_stream(bchip_ctx* c, void** s) {
    CHECK(enter(c));
    if (!s) return fail(BCHIP_E_ARG, "no output pointer");
    *s = (void*)c->stream;
    return BCHIP_OK;
}

int bchip_rope(bchip_ctx* c, float* x, const float* inv_freq, const uint32_t* positions, uint32_t rows,
               uint32_t heads, uint32_t hd, uint32_t rope_dim, uint32_t neox) {
    CHECK(enter(c));
    if (rows == 0 || heads == 0) return BCHIP_OK;
    if (!x || !inv_freq || !positions) return fail(BCHIP_E_ARG, "null pointer");
    if (rope_dim % 2 || rope_dim > hd) return fail(BCHIP_E_ARG, "rope_dim %u for head_dim %u", rope_dim, hd);
    CHECK(check_span(c, x, sat_mul(sat_mul(rows, heads), (uint64_t)hd * 4), "x"));
    CHECK(check_span(c, positions, (uint64_t)rows * 4, "positions"));
    CHECK(check_span(c, inv_freq, (uint64_t)(rope_dim / 2) * 4, "inv_freq"));
    HIP_TRY(rope_launch(x, inv_freq, positions, rows, heads, hd, rope_dim, neox, c->stream), "rope");
    return BCHIP_OK;
}

int bchip_matmul(bchip_ctx* c, const void* w, uint32_t type, const float* x, float* out, uint32_t rows,
                 uint32_t cols, uint32_t n) {
    CHECK(enter(c));
    if (rows == 0 || n == 0) return BCHIP_OK;
    if (!w || !x || !out) return fail(BCHIP_E_ARG, "null pointer");
    uint32_t bw, bb;
    if (!ggml_block(type, bw, bb)) return fail(BCHIP_E_UNSUPPORTED, "ggml type %u", type);
    if (cols == 0 || cols % 32 || cols % bw) return fail(BCHIP_E_ARG, "cols %u: not whole groups of 32 and blocks of %u", cols, bw);
    if ((uintptr_t)w % 16 || (uintptr_t)x % 16) return fail(BCHIP_E_ARG, "w and x must be 16-byte aligned");
    const uint64_t row_bytes = (uint64_t)cols / bw * bb;
    if (row_bytes > UINT32_MAX) return fail(BCHIP_E_ARG, "cols %u: a row of more than 4 GiB", cols);
    if (n > MATMUL_MAX_N) return fail(BCHIP_E_ARG, "%u input rows (at most %u a call)", n, MATMUL_MAX_N);
    CHECK(check_span(c, w, sat_mul(row_bytes, rows), "weights"));
    CHECK(check_span(c, x, sat_mul(n, (uint64_t)cols * 4), "x"));
    CHECK(check_span(c, out, sat_mul(n, (uint64_t)rows * 4), "out"));
    void* scratch = nullptr;
    if (const size_t sb = matmul_scratch_bytes(type, rows, cols, n)) {
        HIP_TRY(c->ws.reserve_vt(sb), "matmul scratch");
        scratch = c->ws.vt;
    }
    HIP_TRY(matmul_launch(w, type, x, out, rows, cols, n, (uint32_t)row_bytes, scratch, c->mm_cnt, c->stream),
            "matmul");
    return BCHIP_OK;
}

int bchip_rms_norm(bchip_ctx* c, const float* x, const float* w, float* out, uint32_t rows, uint32_t cols, float eps) {
    CHECK(enter(c));
    if (rows == 0) return BCHIP_OK;
    if (!x || !w || !out) return fail(BCHIP_E_ARG, "null pointer");
    if (cols == 0) return fail(BCHIP_E_ARG, "cols 0");
    CHECK(check_span(c, x, sat_mul(rows, (uint64_t)cols * 4), "x"));
    CHECK(check_span(c, w, (uint64_t)cols * 4, "w"));
    CHECK(check_span(c, out, sat_mul(rows, (uint64_t)cols * 4), "out"));
    const bool vec = cols % 4 == 0 && ((uintptr_t)x | (uintptr_t)w | (uintptr_t)out) % 16 == 0;
    HIP_TRY(rms_norm_launch(x, w, out, rows, cols, eps, vec, c->stream), "rms_norm");
    return BCHIP_OK;
}

static int elementwise(bchip_ctx* c, int op, float* x, const float* y, uint64_t n, uint32_t dim, uint64_t y_len,
                       const char* what) {
    CHECK(enter(c));
    if (n == 0) return BCHIP_OK;
    if (!x || !y) return fail(BCHIP_E_ARG, "null pointer");
    CHECK(check_span(c, x, sat_mul(n, 4), what));
    CHECK(check_span(c, y, sat_mul(y_len, 4), what));
    HIP_TRY(elementwise_launch(op, x, y, n, dim, c->stream), what);
    return BCHIP_OK;
}

int bchip_bias_add(bchip_ctx* c, float* x, const float* b, uint64_t n, uint32_t dim) {
    if (dim == 0) {
        CHECK(enter(c));
        return fail(BCHIP_E_ARG, "bias of dim 0");
    }
    return elementwise(c, EW_BIAS, x, b, n, dim, dim, "bias_add");
}

int bchip_silu_mul(bchip_ctx* c, float* g, const float* u, uint64_t n) {
    return elementwise(c, EW_SILU_MUL, g, u, n, 1, n, "silu_mul");
}

int bchip_add(bchip_ctx* c, float* x, const float* y, uint64_t n) { return elementwise(c, EW_ADD, x, y, n, 1, n, "add"); }

int bchip_copy(bchip_ctx* c, const void* src, uint32_t st, void* dst, uint32_t dt, uint64_t off, uint64_t n) {
    CHECK(enter(c));
    if (n == 0) return BCHIP_OK;
    if (!src || !dst) return fail(BCHIP_E_ARG, "null pointer");
    if (st > 1 || dt > 1) return fail(BCHIP_E_ARG, "element types %u, %u", st, dt);
    CHECK(check_span(c, src, sat_mul(n, esize(st)), "copy source"));
    CHECK(check_at(c, dst, sat_mul(off, esize(dt)), sat_mul(n, esize(dt)), "copy destination"));
    HIP_TRY(copy_launch(src, st, dst, dt, off, n, c->stream), "copy");
    return BCHIP_OK;
}

int bchip_move(bchip_ctx* c, void* buf, uint32_t type, uint64_t from, uint64_t to, uint64_t n) {
    CHECK(enter(c));
    if (n == 0) return BCHIP_OK;
    if (!buf) return fail(BCHIP_E_ARG, "null pointer");
    if (type > 1) return fail(BCHIP_E_ARG, "element type %u", type);
    if (to > from) return fail(BCHIP_E_ARG, "move to %llu after from %llu", (unsigned long long)to,
                                (unsigned long long)from);
    CHECK(check_span(c, buf, sat_mul(sat_add(from, n), esize(type)), "move"));
    HIP_TRY(move_launch(buf, type, from, to, n, c->stream), "move");
    return BCHIP_OK;
}

int bchip_cache_grow(bchip_ctx* c, const void* const* src, void* const* dst, uint32_t nbufs, uint32_t type,
                     uint64_t keep, uint64_t total) {
    CHECK(enter(c));
    if (nbufs == 0 || total == 0) return BCHIP_OK;
    if (!dst || (keep > 0 && !src)) return fail(BCHIP_E_ARG, "null pointer");
    if (type > 1) return fail(BCHIP_E_ARG, "element type %u", type);
    if (keep > total) return fail(BCHIP_E_ARG, "keep %llu past total %llu", (unsigned long long)keep,
                                  (unsigned long long)total);
    const uint64_t kb = sat_mul(keep, esize(type)), tb = sat_mul(total, esize(type));
    for (uint32_t b = 0; b < nbufs; b++) {
        const uint8_t* s = keep > 0 ? (const uint8_t*)src[b] : nullptr;
        const uint8_t* d = (const uint8_t*)dst[b];
        if (!d || (keep > 0 && !s)) return fail(BCHIP_E_ARG, "null buffer %u", b);
        if ((uintptr_t)d % 16 || (uintptr_t)s % 16) return fail(BCHIP_E_ARG, "buffer %u: not 16-byte aligned", b);
        if (s && s < d + tb && d < s + kb) return fail(BCHIP_E_ARG, "buffer %u: source and destination overlap", b);
        if (s) CHECK(check_span(c, s, kb, "grow source"));
        CHECK(check_span(c, d, tb, "grow destination"));
    }
    std::vector<const void*> sv(nbufs, nullptr);
    if (keep > 0)
        for (uint32_t b = 0; b < nbufs; b++) sv[b] = src[b];
    HIP_TRY(grow_launch(sv.data(), dst, nbufs, kb, tb, c->stream), "cache_grow");
    return BCHIP_OK;
}

int bchip_keep(bchip_ctx* c, void* const* bufs, uint32_t nbufs, uint32_t type, uint32_t width, uint64_t base,
               const uint32_t* rows, uint32_t nrows) {
    CHECK(enter(c));
    if (nbufs == 0 || nrows == 0) return BCHIP_OK;
    if (!bufs || !rows) return fail(BCHIP_E_ARG, "null pointer");
    if (type > 1) return fail(BCHIP_E_ARG, "element type %u", type);
    if (nrows > 64) return fail(BCHIP_E_ARG, "%u rows (at most 64)", nrows);
    for (uint32_t i = 0; i + 1 < nrows; i++)
        if (rows[i] >= rows[i + 1]) return fail(BCHIP_E_ARG, "rows are not an ascending path");
    const uint64_t end = sat_mul(sat_mul(sat_add(base, (uint64_t)rows[nrows - 1] + 1), width), esize(type));
    for (uint32_t b = 0; b < nbufs; b++) {
        if (!bufs[b]) return fail(BCHIP_E_ARG, "null buffer %u", b);
        CHECK(check_span(c, bufs[b], end, "keep"));
    }
    HIP_TRY(keep_launch(bufs, nbufs, type, width, base, rows, nrows, c->stream), "keep");
    return BCHIP_OK;
}

int bchip_rope_append(bchip_ctx* c, float* q, const float* k, const float* v, void* kc, void* vc, uint32_t kv_type,
                      const float* inv_freq, const uint32_t* positions, uint32_t rows, uint32_t nh, uint32_t nkv,
                      uint32_t hd, uint32_t rope_dim, uint32_t neox, uint64_t slot0) {
    CHECK(enter(c));
    if (rows == 0) return BCHIP_OK;
    if (!q || !k || !v || !kc || !vc || !inv_freq || !positions) return fail(BCHIP_E_ARG, "null pointer");
    if (kv_type > 1) return fail(BCHIP_E_ARG, "element type %u", kv_type);
    if (hd % 2 || rope_dim % 2 || rope_dim > hd) return fail(BCHIP_E_ARG, "rope_dim %u for head_dim %u", rope_dim, hd);
    if (nh == 0 || nkv == 0) return fail(BCHIP_E_ARG, "no heads");
    const uint64_t kvd = (uint64_t)nkv * hd;
    CHECK(check_span(c, q, sat_mul(sat_mul(rows, nh), (uint64_t)hd * 4), "q"));
    CHECK(check_span(c, k, sat_mul(rows, kvd * 4), "k"));
    CHECK(check_span(c, v, sat_mul(rows, kvd * 4), "v"));
    const uint64_t cache_bytes = sat_mul(sat_mul(sat_add(slot0, rows), kvd), esize(kv_type));
    CHECK(check_span(c, kc, cache_bytes, "kc"));
    CHECK(check_span(c, vc, cache_bytes, "vc"));
    CHECK(check_span(c, positions, (uint64_t)rows * 4, "positions"));
    CHECK(check_span(c, inv_freq, (uint64_t)(rope_dim / 2) * 4, "inv_freq"));
    HIP_TRY(rope_append_launch(q, k, v, kc, vc, kv_type, inv_freq, positions, rows, nh, nkv, hd, rope_dim, neox,
                               slot0, c->stream),
            "rope_append");
    return BCHIP_OK;
}

int bchip_attention(bchip_ctx* c, const float* q, const void* kc, const void* vc, uint32_t kv_type, float* out,
                    const uint32_t* masks, uint32_t tree, uint32_t rows, uint32_t nh, uint32_t nkv, uint32_t hd,
                    uint32_t pos, float scale) {
    CHECK(enter(c));
    if (rows == 0) return BCHIP_OK;
    if (!q || !kc || !vc || !out) return fail(BCHIP_E_ARG, "null pointer");
    if (kv_type > 1) return fail(BCHIP_E_ARG, "element type %u", kv_type);
    CHECK(check_heads(nh, nkv, hd));
    if (!aligned16(q) || !aligned16(out) || !aligned16(kc) || !aligned16(vc))
        return fail(BCHIP_E_ARG, "q, out and the caches must be 16-byte aligned");
    if ((uint64_t)pos + rows > 0xffffffffull) return fail(BCHIP_E_ARG, "position past 2^32");
    if (tree) {
        if (!masks) return fail(BCHIP_E_ARG, "a tree needs its masks");
        if (rows > MAX_ITEMS) return fail(BCHIP_E_ARG, "a tree pass of %u rows (at most %u)", rows, MAX_ITEMS);
        if ((uint64_t)pos + MAX_ITEMS > 0xffffffffull) return fail(BCHIP_E_ARG, "tree slots past 2^32");
        CHECK(check_span(c, masks, (uint64_t)rows * 8, "masks"));
    }
    const uint64_t kvd = (uint64_t)nkv * hd, slots = (uint64_t)pos + rows;
    CHECK(check_span(c, q, sat_mul(sat_mul(rows, nh), (uint64_t)hd * 4), "q"));
    CHECK(check_span(c, out, sat_mul(sat_mul(rows, nh), (uint64_t)hd * 4), "out"));
    CHECK(check_span(c, kc, sat_mul(slots, kvd * esize(kv_type)), "kc"));
    CHECK(check_span(c, vc, sat_mul(slots, kvd * esize(kv_type)), "vc"));
    const uint64_t row_bytes = kvd * esize(kv_type);
    const uint64_t limit = std::min(bytes_left(c, kc), bytes_left(c, vc)) / row_bytes;
    AttnCall a{q, kc, vc, kv_type, out, masks, tree ? 1u : 0u, rows, nh, nkv, hd, pos, scale, limit};
    c->take_marks(a);
    hipError_t e;
    // f32 caches: the f32 path, one arithmetic for every row of every pass.
    // f16 caches: one row: the one-row kernel. Tree rows: each row gathers its own list
    // (decode-kernel units). Lines of two or more rows (prefill, speculative verify): the
    // shared kernels, which read each K/V block once for every row and head of a KV head they
    // hold (split over the list when there are few of them). Every multi-row kernel computes a
    // row with the same arithmetic, so the choice does not change a bit of the result.
    if (kv_type == BCHIP_F32) {
        e = f32_attention(a, 0, c->ws, c->stream);
    } else if (rows == 1 && !tree) {
        Item item{};
        item.row = 0;
        item.nrows = 1;
        item.len = (uint32_t)slots;
        e = row_attention(a, &item, 1, c->ws, c->stream);
    } else if (tree) {
        // A row's list is pos + popcount(its mask), and a tree grown a level at a time holds
        // more nodes than the pass has rows (Shape::new, model.rs:421-443): a row's mask may
        // name any of slots pos .. pos + 63. The chunks cover that farthest list; a chunk
        // past a row's own list computes nothing and leaves an empty state, which the fold
        // takes as the identity (weight 0, the running state's weight exactly 1).
        const uint64_t far = (uint64_t)pos + MAX_ITEMS;
        Item items[MAX_ITEMS];
        for (uint32_t i = 0; i < rows; i++) {
            Item& I = items[i];
            I = Item{};
            I.row = i;
            I.nrows = 1;
            I.len = (uint32_t)std::min<uint64_t>(far, 0xffffffffull);
            I.nchunk = (uint32_t)((far + CHUNK_MULTI - 1) / CHUNK_MULTI);
            I.chunk = CHUNK_MULTI;
        }
        e = direct_attention(a, items, rows, c->ws, c->stream);
    } else {
        e = shared_attention(a, c->ws, c->stream);
    }
    HIP_TRY(e, "attention");
    return BCHIP_OK;
}

int bchip_rope_append_attention_rows(bchip_ctx* c, float* q, const float* k, const float* v, void* kc, void* vc,
                                     uint32_t kv_type, const float* inv_freq, const uint32_t* positions,
                                     uint32_t rows, uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t rope_dim,
                                     uint32_t neox, uint32_t pos, float scale, float* out) {
    CHECK(enter(c));
    if (rows == 0) return BCHIP_OK;
    if (!q || !k || !v || !kc || !vc || !inv_freq || !positions || !out) return fail(BCHIP_E_ARG, "null pointer");
    if (kv_type > 1) return fail(BCHIP_E_ARG, "element type %u", kv_type);
    CHECK(check_heads(nh, nkv, hd));
    if (rope_dim % 2 || rope_dim > hd) return fail(BCHIP_E_ARG, "rope_dim %u for head_dim %u", rope_dim, hd);
    if (!aligned16(q) || !aligned16(out) || !aligned16(kc) || !aligned16(vc))
        return fail(BCHIP_E_ARG, "q, out and the caches must be 16-byte aligned");
    if ((uint64_t)pos + rows > 0xffffffffull) return fail(BCHIP_E_ARG, "position past 2^32");
    const uint64_t kvd = (uint64_t)nkv * hd, slots = (uint64_t)pos + rows;
    CHECK(check_span(c, q, sat_mul(sat_mul(rows, nh), (uint64_t)hd * 4), "q"));
    CHECK(check_span(c, out, sat_mul(sat_mul(rows, nh), (uint64_t)hd * 4), "out"));
    CHECK(check_span(c, k, sat_mul(rows, kvd * 4), "k"));
    CHECK(check_span(c, v, sat_mul(rows, kvd * 4), "v"));
    CHECK(check_span(c, kc, sat_mul(slots, kvd * esize(kv_type)), "kc"));
    CHECK(check_span(c, vc, sat_mul(slots, kvd * esize(kv_type)), "vc"));
    CHECK(check_span(c, positions, (uint64_t)rows * 4, "positions"));
    CHECK(check_span(c, inv_freq, (uint64_t)(rope_dim / 2) * 4, "inv_freq"));
    if (kv_type == BCHIP_F32 && rows <= 8) {
        // f32 caches: attn_f32 rotates q and appends the new rows itself (the two calls' bits).
        const uint64_t limit = std::min(bytes_left(c, kc), bytes_left(c, vc)) / (kvd * esize(kv_type));
        AttnCall a{q, kc, vc, kv_type, out, nullptr, 0u, rows, nh, nkv, hd, pos, scale, limit};
        const RopeArgs r{q, k, v, inv_freq, positions, rope_dim, neox};
        c->take_marks(a);
        HIP_TRY(f32_attention(a, 0, c->ws, c->stream, &r), "rope_append_attention_rows");
        return BCHIP_OK;
    }
    // (The one-launch form loads the new k and v rows 16 bytes a lane.)
    if (kv_type == BCHIP_F16 && rows > 1 && aligned16(k) && aligned16(v)) {
        const uint64_t limit = std::min(bytes_left(c, kc), bytes_left(c, vc)) / (kvd * esize(kv_type));
        AttnCall a{q, kc, vc, kv_type, out, nullptr, 0u, rows, nh, nkv, hd, pos, scale, limit};
        const RopeArgs r{q, k, v, inv_freq, positions, rope_dim, neox};
        c->take_marks(a);
        const hipError_t e = shared_attention_fused(a, r, c->ws, c->stream);
        if (e != hipErrorNotSupported) {
            HIP_TRY(e, "rope_append_attention_rows");
            return BCHIP_OK;
        }
        c->restore_marks(a);
    }
    // Shapes the fused launch does not take: the two calls.
    HIP_TRY(rope_append_launch(q, k, v, kc, vc, kv_type, inv_freq, positions, rows, nh, nkv, hd, rope_dim, neox, pos,
                               c->stream),
            "rope_append");
    return bchip_attention(c, q, kc, vc, kv_type, out, nullptr, 0, rows, nh, nkv, hd, pos, scale);
}

// bchip_rope_append_attention on workspace ws; with a fixed workspace (the no-allocation
// entry point) every launch's scratch is checked to fit before anything is launched.
static int fused_step(bchip_ctx* c, Workspace& ws, float* q, const float* k, const float* v, void* kc, void* vc,
                      uint32_t kv_type, const float* inv_freq, const uint32_t* positions, uint32_t nh,
                      uint32_t nkv, uint32_t hd, uint32_t rope_dim, uint32_t neox, uint32_t pos, float scale,
                      float* out) {
    CHECK(enter(c));
    if (!q || !k || !v || !kc || !vc || !inv_freq || !positions || !out) return fail(BCHIP_E_ARG, "null pointer");
    if (kv_type > 1) return fail(BCHIP_E_ARG, "element type %u", kv_type);
    CHECK(check_heads(nh, nkv, hd));
    if (rope_dim % 2 || rope_dim > hd) return fail(BCHIP_E_ARG, "rope_dim %u for head_dim %u", rope_dim, hd);
    const bool fuse = kv_type == BCHIP_F16 && row_fusable(nh, nkv, hd, rope_dim, neox);
    if (!aligned16(q) || !aligned16(out) || !aligned16(kc) || !aligned16(vc) || (fuse && (!aligned16(k) || !aligned16(v))))
        return fail(BCHIP_E_ARG, "q, k, v, out and the caches must be 16-byte aligned");
    if ((uint64_t)pos + 1 > 0xffffffffull) return fail(BCHIP_E_ARG, "position past 2^32");
    const uint64_t kvd = (uint64_t)nkv * hd, slots = (uint64_t)pos + 1;
    CHECK(check_span(c, q, sat_mul(nh, (uint64_t)hd * 4), "q"));
    CHECK(check_span(c, out, sat_mul(nh, (uint64_t)hd * 4), "out"));
    CHECK(check_span(c, k, kvd * 4, "k"));
    CHECK(check_span(c, v, kvd * 4, "v"));
    CHECK(check_span(c, kc, sat_mul(slots, kvd * esize(kv_type)), "kc"));
    CHECK(check_span(c, vc, sat_mul(slots, kvd * esize(kv_type)), "vc"));
    CHECK(check_span(c, positions, 4, "positions"));
    CHECK(check_span(c, inv_freq, (uint64_t)(rope_dim / 2) * 4, "inv_freq"));
    if (ws.fixed && kv_type == BCHIP_F16) {
        const size_t hdp = hd <= 32 ? 32 : hd <= 64 ? 64 : hd <= 128 ? 128 : 256;
        const size_t need = row_state_slots(slots, nkv);
        if (need * hdp * 4 > ws.o_cap || need * 8 > ws.ml_cap || (fuse && (size_t)nh * hd * 4 > ws.qrot_cap))
            return fail(BCHIP_E_ARG,
                        "this step takes %zu bytes of chunk states and %zu of staged q; the no-allocation "
                        "entry point holds %zu and %zu",
                        need * hdp * 4, fuse ? (size_t)nh * hd * 4 : (size_t)0, ws.o_cap, ws.qrot_cap);
    }
    const uint64_t limit = std::min(bytes_left(c, kc), bytes_left(c, vc)) / (kvd * esize(kv_type));
    AttnCall a{q, kc, vc, kv_type, out, nullptr, 0u, 1u, nh, nkv, hd, pos, scale, limit};
    c->take_marks(a);
    if (kv_type == BCHIP_F32) {
        // f32 caches: attn_f32 rotates q and appends the new row itself (the two calls' bits).
        const RopeArgs r{q, k, v, inv_freq, positions, rope_dim, neox};
        HIP_TRY(f32_attention(a, 0, ws, c->stream, &r), "rope_append_attention");
        return BCHIP_OK;
    }
    if (!fuse) {
        // Shapes the fused kernel does not take: the two calls.
        HIP_TRY(rope_append_launch(q, k, v, kc, vc, kv_type, inv_freq, positions, 1, nh, nkv, hd, rope_dim, neox,
                                   pos, c->stream),
                "rope_append");
        Item item{};
        item.row = 0;
        item.nrows = 1;
        item.len = (uint32_t)slots;
        HIP_TRY(row_attention(a, &item, 1, ws, c->stream), "attention");
        return BCHIP_OK;
    }
    RopeArgs r{q, k, v, inv_freq, positions, rope_dim, neox};
    HIP_TRY(row_attention_fused(a, r, ws, c->stream), "rope_append_attention");
    return BCHIP_OK;
}

int bchip_rope_append_attention(bchip_ctx* c, float* q, const float* k, const float* v, void* kc, void* vc,
                                uint32_t kv_type, const float* inv_freq, const uint32_t* positions, uint32_t nh,
                                uint32_t nkv, uint32_t hd, uint32_t rope_dim, uint32_t neox, uint32_t pos,
                                float scale, float* out) {
    if (!c) return fail(BCHIP_E_ARG, "no context");
    return fused_step(c, c->ws, q, k, v, kc, vc, kv_type, inv_freq, positions, nh, nkv, hd, rope_dim, neox, pos,
                      scale, out);
}

int bchip_rope_append_attention_noalloc(bchip_ctx* c, float* q, const float* k, const float* v, void* kc, void* vc,
                                        uint32_t kv_type, const float* inv_freq, const uint32_t* positions,
                                        uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t rope_dim, uint32_t neox,
                                        uint32_t pos, float scale, float* out) {
    if (!c) return fail(BCHIP_E_ARG, "no context");
    return fused_step(c, c->fixed_ws, q, k, v, kc, vc, kv_type, inv_freq, positions, nh, nkv, hd, rope_dim, neox,
                      pos, scale, out);
}

// Checks shared by the ragged calls: every sequence sees at least one slot, and its slots
// lie inside both caches.
static int check_ragged(bchip_ctx* c, const void* kc, const void* vc, uint32_t kv_type, const uint32_t* seq_lens,
                        const uint64_t* kv_offsets, uint32_t nseq, uint64_t kvd) {
    if (nseq > 256) return fail(BCHIP_E_ARG, "%u sequences (at most 256)", nseq);
    for (uint32_t i = 0; i < nseq; i++) {
        if (seq_lens[i] == 0) return fail(BCHIP_E_ARG, "sequence %u sees no slots", i);
        const uint64_t end = sat_mul(sat_mul(sat_add(kv_offsets[i], seq_lens[i]), kvd), esize(kv_type));
        CHECK(check_span(c, kc, end, "kc"));
        CHECK(check_span(c, vc, end, "vc"));
    }
    return BCHIP_OK;
}

// The attention of a ragged batch, arguments checked: sequence i's row of q against its
// seq_lens[i] slots from kv_offsets[i].
static int ragged_attention(bchip_ctx* c, AttnCall& a, const uint32_t* seq_lens, const uint64_t* kv_offsets,
                            uint32_t nseq) {
    const float* q = a.q;
    float* out = a.out;
    const uint32_t nh = a.nh, nkv = a.nkv, hd = a.hd;
    if (a.kv_type == BCHIP_F32) {
        // One f32-path call per sequence, each at its place in the pool, its result the bits of
        // the sequence alone. The workspace is sized for the longest first, so that no call
        // reallocates it while an earlier one may still read it.
        uint32_t longest = 0;
        for (uint32_t i = 0; i < nseq; i++) longest = std::max(longest, seq_lens[i]);
        const size_t most = (size_t)nkv * ((longest + CHUNK_MULTI - 1) / CHUNK_MULTI) * 16;
        HIP_TRY(c->ws.reserve(most, hd <= 32 ? 32 : hd <= 64 ? 64 : hd <= 128 ? 128 : 256), "workspace");
        for (uint32_t i = 0; i < nseq; i++) {
            AttnCall ai = a;
            ai.q = q + (size_t)i * nh * hd;
            ai.out = out + (size_t)i * nh * hd;
            ai.pos = seq_lens[i] - 1;
            if (i > 0) ai.ev_before = ai.ev_after = nullptr;
            HIP_TRY(f32_attention(ai, kv_offsets[i], c->ws, c->stream), "ragged attention");
        }
        return BCHIP_OK;
    }
    for (uint32_t s0 = 0; s0 < nseq; s0 += MAX_ITEMS) {
        const uint32_t ns = std::min<uint32_t>(MAX_ITEMS, nseq - s0);
        Item items[MAX_ITEMS];
        for (uint32_t i = 0; i < ns; i++) {
            Item& I = items[i];
            I = Item{};
            I.row = s0 + i;
            I.nrows = 1;
            I.len = seq_lens[s0 + i];
            I.kvoff = kv_offsets[s0 + i];
        }
        HIP_TRY(row_attention(a, items, ns, c->ws, c->stream), "ragged attention");
        a.ev_before = a.ev_after = nullptr;  // the events mark the first launch only
    }
    return BCHIP_OK;
}

int bchip_attention_ragged(bchip_ctx* c, const float* q, const void* kc, const void* vc, uint32_t kv_type,
                           float* out, const uint32_t* seq_lens, const uint64_t* kv_offsets, uint32_t nseq,
                           uint32_t nh, uint32_t nkv, uint32_t hd, float scale) {
    CHECK(enter(c));
    if (nseq == 0) return BCHIP_OK;
    if (!q || !kc || !vc || !out || !seq_lens || !kv_offsets) return fail(BCHIP_E_ARG, "null pointer");
    if (kv_type > 1) return fail(BCHIP_E_ARG, "element type %u", kv_type);
    CHECK(check_heads(nh, nkv, hd));
    if (!aligned16(q) || !aligned16(out) || !aligned16(kc) || !aligned16(vc))
        return fail(BCHIP_E_ARG, "q, out and the caches must be 16-byte aligned");
    const uint64_t kvd = (uint64_t)nkv * hd;
    CHECK(check_span(c, q, sat_mul(sat_mul(nseq, nh), (uint64_t)hd * 4), "q"));
    CHECK(check_span(c, out, sat_mul(sat_mul(nseq, nh), (uint64_t)hd * 4), "out"));
    CHECK(check_ragged(c, kc, vc, kv_type, seq_lens, kv_offsets, nseq, kvd));
    const uint64_t limit = std::min(bytes_left(c, kc), bytes_left(c, vc)) / (kvd * esize(kv_type));
    AttnCall a{q, kc, vc, kv_type, out, nullptr, 0u, 1u, nh, nkv, hd, 0u, scale, limit};
    c->take_marks(a);
    return ragged_attention(c, a, seq_lens, kv_offsets, nseq);
}

int bchip_rope_append_ragged(bchip_ctx* c, float* q, const float* k, const float* v, void* kc, void* vc,
                             uint32_t kv_type, const float* inv_freq, const uint32_t* positions,
                             const uint32_t* seq_lens, const uint64_t* kv_offsets, uint32_t nseq, uint32_t nh,
                             uint32_t nkv, uint32_t hd, uint32_t rope_dim, uint32_t neox) {
    CHECK(enter(c));
    if (nseq == 0) return BCHIP_OK;
    if (!q || !k || !v || !kc || !vc || !inv_freq || !positions || !seq_lens || !kv_offsets)
        return fail(BCHIP_E_ARG, "null pointer");
    if (kv_type > 1) return fail(BCHIP_E_ARG, "element type %u", kv_type);
    if (hd % 2 || rope_dim % 2 || rope_dim > hd) return fail(BCHIP_E_ARG, "rope_dim %u for head_dim %u", rope_dim, hd);
    if (nh == 0 || nkv == 0) return fail(BCHIP_E_ARG, "no heads");
    const uint64_t kvd = (uint64_t)nkv * hd;
    CHECK(check_span(c, q, sat_mul(sat_mul(nseq, nh), (uint64_t)hd * 4), "q"));
    CHECK(check_span(c, k, sat_mul(nseq, kvd * 4), "k"));
    CHECK(check_span(c, v, sat_mul(nseq, kvd * 4), "v"));
    CHECK(check_span(c, positions, (uint64_t)nseq * 4, "positions"));
    CHECK(check_span(c, inv_freq, (uint64_t)(rope_dim / 2) * 4, "inv_freq"));
    CHECK(check_ragged(c, kc, vc, kv_type, seq_lens, kv_offsets, nseq, kvd));
    std::vector<uint64_t> slots(nseq);
    for (uint32_t i = 0; i < nseq; i++) slots[i] = kv_offsets[i] + seq_lens[i] - 1;
    HIP_TRY(rope_append_ragged_launch(q, k, v, kc, vc, kv_type, inv_freq, positions, nseq, nh, nkv, hd, rope_dim,
                                      neox, slots.data(), c->stream),
            "rope_append_ragged");
    return BCHIP_OK;
}

int bchip_rope_append_attention_ragged(bchip_ctx* c, float* q, const float* k, const float* v, void* kc, void* vc,
                                       uint32_t kv_type, const float* inv_freq, const uint32_t* positions,
                                       const uint32_t* seq_lens, const uint64_t* kv_offsets, uint32_t nseq,
                                       uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t rope_dim, uint32_t neox,
                                       float scale, float* out) {
    CHECK(enter(c));
    if (nseq == 0) return BCHIP_OK;
    if (!q || !k || !v || !kc || !vc || !inv_freq || !positions || !seq_lens || !kv_offsets || !out)
        return fail(BCHIP_E_ARG, "null pointer");
    if (kv_type > 1) return fail(BCHIP_E_ARG, "element type %u", kv_type);
    CHECK(check_heads(nh, nkv, hd));
    if (rope_dim % 2 || rope_dim > hd) return fail(BCHIP_E_ARG, "rope_dim %u for head_dim %u", rope_dim, hd);
    const bool fuse = kv_type == BCHIP_F16 && row_fusable(nh, nkv, hd, rope_dim, neox);
    if (!aligned16(q) || !aligned16(out) || !aligned16(kc) || !aligned16(vc) || (fuse && (!aligned16(k) || !aligned16(v))))
        return fail(BCHIP_E_ARG, "q, k, v, out and the caches must be 16-byte aligned");
    const uint64_t kvd = (uint64_t)nkv * hd;
    CHECK(check_span(c, q, sat_mul(sat_mul(nseq, nh), (uint64_t)hd * 4), "q"));
    CHECK(check_span(c, out, sat_mul(sat_mul(nseq, nh), (uint64_t)hd * 4), "out"));
    CHECK(check_span(c, k, sat_mul(nseq, kvd * 4), "k"));
    CHECK(check_span(c, v, sat_mul(nseq, kvd * 4), "v"));
    CHECK(check_span(c, positions, (uint64_t)nseq * 4, "positions"));
    CHECK(check_span(c, inv_freq, (uint64_t)(rope_dim / 2) * 4, "inv_freq"));
    CHECK(check_ragged(c, kc, vc, kv_type, seq_lens, kv_offsets, nseq, kvd));
    const uint64_t limit = std::min(bytes_left(c, kc), bytes_left(c, vc)) / (kvd * esize(kv_type));
    AttnCall a{q, kc, vc, kv_type, out, nullptr, 0u, 1u, nh, nkv, hd, 0u, scale, limit};
    c->take_marks(a);
    if (!fuse) {
        // f32 caches, and shapes the fused kernel does not take: the two calls.
        std::vector<uint64_t> slots(nseq);
        for (uint32_t i = 0; i < nseq; i++) slots[i] = kv_offsets[i] + seq_lens[i] - 1;
        HIP_TRY(rope_append_ragged_launch(q, k, v, kc, vc, kv_type, inv_freq, positions, nseq, nh, nkv, hd,
                                          rope_dim, neox, slots.data(), c->stream),
                "rope_append_ragged");
        return ragged_attention(c, a, seq_lens, kv_offsets, nseq);
    }
    RopeArgs r{q, k, v, inv_freq, positions, rope_dim, neox};
    for (uint32_t s0 = 0; s0 < nseq; s0 += MAX_ITEMS) {
        const uint32_t ns = std::min<uint32_t>(MAX_ITEMS, nseq - s0);
        Item items[MAX_ITEMS];
        for (uint32_t i = 0; i < ns; i++) {
            Item& I = items[i];
            I = Item{};
            I.row = s0 + i;
            I.nrows = 1;
            I.len = seq_lens[s0 + i];
            I.kvoff = kv_offsets[s0 + i];
        }
        HIP_TRY(row_attention_fused_items(a, r, items, ns, c->ws, c->stream), "rope_append_attention_ragged");
        a.ev_before = a.ev_after = nullptr;
    }
    return BCHIP_OK;
}

int bchip_sample(bchip_ctx* c, const float* scores, uint32_t rows, uint32_t vocab, float temperature, float top_p,
                 uint64_t seed, uint64_t step0, uint32_t* ids) {
    CHECK(enter(c));
    if (rows == 0) return BCHIP_OK;
    if (!scores || !ids) return fail(BCHIP_E_ARG, "null pointer");
    if (vocab == 0) return fail(BCHIP_E_ARG, "an empty vocabulary");
    if (rows > 65535) return fail(BCHIP_E_ARG, "%u rows (at most 65535 a call)", rows);
    CHECK(check_span(c, scores, sat_mul(rows, (uint64_t)vocab * 4), "scores"));
    CHECK(check_span(c, ids, (uint64_t)rows * 4, "ids"));
    size_t need = 0;
    if (temperature > 0.0f) {
        need = sample_scratch_bytes(rows, vocab);
        HIP_TRY(c->ws.reserve_vt(need), "sampler scratch");
    }
    HIP_TRY(sample_launch(scores, rows, vocab, temperature, top_p, seed, step0, ids, c->ws.vt, c->ws.vt_bytes,
                          c->stream),
            "sample");
    return BCHIP_OK;
}

int bchip_fill_normal(bchip_ctx* c, void* dst, uint32_t type, uint64_t n, uint64_t seed) {
    CHECK(enter(c));
    if (n == 0) return BCHIP_OK;
    if (!dst) return fail(BCHIP_E_ARG, "null pointer");
    if (type > 1) return fail(BCHIP_E_ARG, "element type %u", type);
    CHECK(check_span(c, dst, sat_mul(n, esize(type)), "fill"));
    HIP_TRY(fill_normal_launch(dst, type, n, seed, c->stream), "fill_normal");
    return BCHIP_OK;
}

int bchip_timer_start(bchip_ctx* c) {
    CHECK(enter(c));
    HIP_TRY(hipEventRecord(c->t0, c->stream), "hipEventRecord");
    return BCHIP_OK;
}

int bchip_timer_arm(bchip_ctx* c, void* before, void* after) {
    CHECK(enter(c));
    if (!before || !after) return fail(BCHIP_E_ARG, "null event");
    c->arm_before = (hipEvent_t)before;
    c->arm_after = (hipEvent_t)after;
    return BCHIP_OK;
}

int bchip_timer_stop(bchip_ctx* c, float* ms) {
    CHECK(enter(c));
    if (!ms) return fail(BCHIP_E_ARG, "no output pointer");
    HIP_TRY(hipEventRecord(c->t1, c->stream), "hipEventRecord");
    HIP_TRY(hipEventSynchronize(c->t1), "hipEventSynchronize");
    HIP_TRY(hipEventElapsedTime(ms, c->t0, c->t1), "hipEventElapsedTime");
    return BCHIP_OK;
}

}  // extern "C"
