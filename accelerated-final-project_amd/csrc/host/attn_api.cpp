// C-ABI host layer: validation, positional-encoding tables, scratch memory,
// dispatch onto the HIP kernels, and the reference-compatible drop-in entry
// points (synchronous, exit on error).
//
// Validation runs before any HIP call, so every argument error is reported
// (and testable) without a GPU.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <ctime>
#include <unistd.h>
#include <algorithm>
#include <atomic>
#include <map>
#include <memory>
#include <mutex>
#include <tuple>
#include <vector>

#include "../kernels/launch.hpp"
#include "attn_mi355x.h"

namespace {

thread_local int g_last_hip_error = 0;

int hip_fail(hipError_t e) {
    g_last_hip_error = (int)e;
    return ATN_ERR_HIP;
}

#define ATN_HIP(call)                                  \
    do {                                               \
        hipError_t e_ = (call);                        \
        if (e_ != hipSuccess) return hip_fail(e_);     \
    } while (0)

// ---------------------------------------------------------------- tuning
// The process-wide overrides (atn_set_tuning_ex): an immutable snapshot
// behind an atomic pointer, so that every call reads them without a lock.
// Replaced snapshots are kept (a concurrent call may still read one); they
// are a few dozen bytes each and replaced only by tests and measurement.
std::atomic<const atn_tuning*> g_tune{new atn_tuning{}};
std::vector<std::unique_ptr<const atn_tuning>> g_tune_old;
std::mutex g_tune_mu;

const atn_tuning& tune() { return *g_tune.load(std::memory_order_acquire); }

// Synchronous drop-in calls rerun without the single-launch kernel.
std::atomic<long> g_reruns{0};

// ---------------------------------------------------------------- validation
bool mul_ok(int64_t a, int64_t b, int64_t* out) {
    if (a < 0 || b < 0) return false;
    if (a != 0 && b > INT64_MAX / a) return false;
    *out = a * b;
    return true;
}

struct Shape {
    int B, H, Lq, Lk, D;
    int64_t BH, nq, nk;  // element counts of Q/out and of K/V
};

int check_shape(int B, int H, int Lq, int Lk, int D, Shape* s) {
    if (B < 1 || H < 1 || Lq < 1 || Lk < 1 || D < 1) return ATN_ERR_BAD_DIMENSION;
    int64_t bh, t;
    if (!mul_ok(B, H, &bh)) return ATN_ERR_SIZE_OVERFLOW;
    if (!mul_ok(bh, Lq, &t) || !mul_ok(t, D, &s->nq)) return ATN_ERR_SIZE_OVERFLOW;
    if (!mul_ok(bh, Lk, &t) || !mul_ok(t, D, &s->nk)) return ATN_ERR_SIZE_OVERFLOW;
    if (s->nq > (INT64_MAX / 8) || s->nk > (INT64_MAX / 8)) return ATN_ERR_SIZE_OVERFLOW;
    // The kernels index rows of one head with 32-bit ints.
    if ((int64_t)Lq * D > INT32_MAX || (int64_t)Lk * D > INT32_MAX) return ATN_ERR_SIZE_OVERFLOW;
    s->B = B; s->H = H; s->Lq = Lq; s->Lk = Lk; s->D = D; s->BH = bh;
    return ATN_OK;
}

bool overlaps(const void* a, int64_t abytes, const void* b, int64_t bbytes) {
    const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
    return x < y + (uintptr_t)bbytes && y < x + (uintptr_t)abytes;
}

size_t elem_size(int dtype) { return dtype == ATN_DTYPE_F32 ? 4 : 2; }

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// ---------------------------------------------------------------- resolved encoding
struct PePlan {
    int pek = atn::kPeNone;   // kernel template selector
    atn::PeSide q{}, k{};
    int rotary = 0;
    float base = 10000.0f;
    int pairing = ATN_ROPE_INTERLEAVED;
    bool caller_tables = false;
    // the call may not take the single-launch kernel (a synchronous call's
    // second attempt after that kernel's exchange timed out)
    bool no_fused = false;
    bool no_flash = false;  // nor the flash kernel (atn_tuning.no_flash)
};

int check_pe(const atn_pe_desc* pe, int D, PePlan* plan) {
    *plan = PePlan{};
    if (pe == nullptr || pe->kind == ATN_PE_NONE) return ATN_OK;
    if (pe->kind == ATN_PE_ROPE) {
        const int r = pe->rotary_dim == 0 ? D : pe->rotary_dim;
        if (r < 2 || r > D || (r & 1)) return ATN_ERR_BAD_ROTARY;
        if (pe->pairing != ATN_ROPE_INTERLEAVED && pe->pairing != ATN_ROPE_HALF)
            return ATN_ERR_BAD_ARGUMENT;
        if ((pe->table_a == nullptr) != (pe->table_b == nullptr)) return ATN_ERR_NULL_POINTER;
        const float base = pe->base == 0.0f ? 10000.0f : pe->base;
        if (!(base > 0.0f) || !std::isfinite(base)) return ATN_ERR_BAD_ARGUMENT;
        plan->pek = pe->pairing == ATN_ROPE_HALF ? atn::kPeRopeHalf : atn::kPeRopeInterleaved;
        plan->rotary = r;
        plan->base = base;
        plan->pairing = pe->pairing;
    } else if (pe->kind == ATN_PE_SINUSOIDAL) {
        if ((pe->table_a == nullptr) != (pe->table_b == nullptr)) return ATN_ERR_NULL_POINTER;
        plan->pek = atn::kPeSinusoidal;
        plan->rotary = D;
    } else {
        return ATN_ERR_BAD_ARGUMENT;
    }
    plan->caller_tables = pe->table_a != nullptr;
    plan->q.on = pe->apply_q ? 1 : 0;
    plan->k.on = pe->apply_k ? 1 : 0;
    plan->q.rotary = plan->k.rotary = plan->rotary;
    return ATN_OK;
}

// ---------------------------------------------------------------- per-device state
struct Table {
    float* a = nullptr;
    float* b = nullptr;
    int npos = 0;
    int nfreq = 0;
    bool captured = false;  // bound by a call under stream capture at least once
};

// Library-managed scratch, one per (device, stream) so that calls on
// different streams never share partial results or epoch words.  It is
// zero-filled when allocated.
struct Workspace {
    void* ptr = nullptr;
    size_t bytes = 0;
    bool captured = false;  // enqueued into a stream capture at least once
};

// fp16 encoding tables of the GEMM path's fused K encoding, [npos][D]
// 16-bit units: sinusoidal PE values, or (cos, sin) words per rotation pair.
struct Table16 {
    uint16_t* p = nullptr;
    int npos = 0;
    bool captured = false;
};

struct DeviceState {
    std::map<hipStream_t, Workspace> ws;
    // Superseded library workspaces and tables that captured work used: HIP
    // graphs keep their device addresses, so they are freed only by
    // atn_release_ex (or with the process).  Buffers no capture used are
    // freed when superseded.
    std::vector<std::pair<void*, size_t>> retired;
    size_t live_bytes = 0;  // workspaces and tables in use
    std::map<std::tuple<int, int, uint32_t>, Table> tables;  // (kind, dim, base bits)
    std::map<std::tuple<int, int, int, uint32_t>, Table16> tables16;  // (kind, D, rotary, base)
    int cus = 0;
    int xccs = 0;  // XCDs the device reports (8 on a whole MI355X)
    std::map<std::pair<int, int>, int> fused_per_cu;  // (dtype, LDS bytes) -> workgroups per CU
    // Two pinned host words that receive the status words of the null
    // stream's library workspace and of the allocation-free scratch behind
    // each synchronous drop-in call (allocated once, kept).
    int* status_host = nullptr;
};

std::mutex g_mu;
std::map<int, DeviceState> g_dev;

int current_device(int* dev) {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
        g_last_hip_error = (int)e;
        return ATN_ERR_NO_DEVICE;
    }
    ATN_HIP(hipGetDevice(dev));
    return ATN_OK;
}

// Library allocations (first use or growth of a workspace or table) are
// synchronous and cannot be recorded into a graph: while `stream` is being
// captured they are refused with ATN_ERR_CAPTURE.
int refuse_if_capturing(hipStream_t stream) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    ATN_HIP(hipStreamIsCapturing(stream, &cs));
    return cs == hipStreamCaptureStatusNone ? ATN_OK : ATN_ERR_CAPTURE;
}

bool is_capturing(hipStream_t stream) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

// Growth of a library buffer: at least double the old size, so that the
// superseded buffers of a growing sequence of shapes add up to less than
// the final one.
size_t grown(size_t old_bytes, size_t need) { return std::max(need, 2 * old_bytes); }

// A superseded library buffer: freed once the work that may use it has
// drained (`stream`'s, or the device's for tables shared by every stream),
// unless captured work used it, which keeps it until atn_release_ex.
// Called only outside capture.  Caller holds g_mu.
int supersede(DeviceState& ds, void* p, size_t bytes, bool captured, hipStream_t stream,
              bool device_wide) {
    if (p == nullptr) return ATN_OK;
    ds.live_bytes -= std::min(ds.live_bytes, bytes);
    if (captured) {
        ds.retired.emplace_back(p, bytes);
        return ATN_OK;
    }
    ATN_HIP(device_wide ? hipDeviceSynchronize() : hipStreamSynchronize(stream));
    ATN_HIP(hipFree(p));
    return ATN_OK;
}

// Host-side angle tables with the reference CPU path's float expressions
// (final/rope.cu:27-33, final/sinusoidal.cu:846-851), compact layout
// [pos][nfreq]: RoPE a = cos, b = sin; sinusoidal a = sin, b = cos.
void build_rope_table(std::vector<float>& a, std::vector<float>& b, int npos, int r, float base) {
    const int nf = r / 2;
    std::vector<float> freq(nf);
    for (int i = 0; i < nf; i++) freq[i] = 1.0f / powf(base, (2.0f * i) / r);
    a.resize((size_t)npos * nf);
    b.resize((size_t)npos * nf);
    for (int pos = 0; pos < npos; pos++)
        for (int i = 0; i < nf; i++) {
            const float theta = pos * freq[i];
            a[(size_t)pos * nf + i] = cosf(theta);
            b[(size_t)pos * nf + i] = sinf(theta);
        }
}

void build_sin_table(std::vector<float>& a, std::vector<float>& b, int npos, int D) {
    const int nf = (D + 1) / 2;
    std::vector<float> freq(nf);
    for (int f = 0; f < nf; f++) freq[f] = 1.0f / powf(10000.0f, (2.0f * f) / (float)D);
    a.resize((size_t)npos * nf);
    b.resize((size_t)npos * nf);
    for (int pos = 0; pos < npos; pos++)
        for (int f = 0; f < nf; f++) {
            const float angle = pos * freq[f];
            a[(size_t)pos * nf + f] = sinf(angle);
            b[(size_t)pos * nf + f] = cosf(angle);
        }
}

// Returns the device tables for this encoding, building or growing them
// (synchronously) when needed.  Caller holds g_mu.
int get_table(DeviceState& ds, const PePlan& plan, int D, int npos, hipStream_t stream,
              bool no_alloc, Table** out) {
    const bool rope = plan.pek != atn::kPeSinusoidal;
    uint32_t base_bits;
    std::memcpy(&base_bits, &plan.base, 4);
    const auto key = std::make_tuple(rope ? 1 : 2, rope ? plan.rotary : D, rope ? base_bits : 0u);
    Table& t = ds.tables[key];
    if (t.a == nullptr || t.npos < npos) {
        if (no_alloc) return ATN_ERR_NOT_PREPARED;
        int st = refuse_if_capturing(stream);
        if (st != ATN_OK) return st;
        const int want = std::max({64, npos, t.a ? 2 * t.npos : 0});
        std::vector<float> a, b;
        int nf;
        if (rope) {
            build_rope_table(a, b, want, plan.rotary, plan.base);
            nf = plan.rotary / 2;
        } else {
            build_sin_table(a, b, want, D);
            nf = (D + 1) / 2;
        }
        if (t.a) {
            const size_t old = (size_t)t.npos * t.nfreq * sizeof(float);
            st = supersede(ds, t.a, old, t.captured, stream, true);
            if (st == ATN_OK) st = supersede(ds, t.b, old, t.captured, stream, true);
            t.a = t.b = nullptr;
            t.captured = false;
            if (st != ATN_OK) return st;
        }
        const size_t bytes = a.size() * sizeof(float);
        ATN_HIP(hipMalloc(&t.a, bytes));
        ATN_HIP(hipMalloc(&t.b, bytes));
        ds.live_bytes += 2 * bytes;
        ATN_HIP(hipMemcpy(t.a, a.data(), bytes, hipMemcpyHostToDevice));
        ATN_HIP(hipMemcpy(t.b, b.data(), bytes, hipMemcpyHostToDevice));
        t.npos = want;
        t.nfreq = nf;
    }
    *out = &t;
    return ATN_OK;
}

uint16_t f16_bits(float x) {
    const _Float16 h = (_Float16)x;  // nearest even
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}

// The GEMM path's fp16 tables, from the same float expressions as the fp32
// tables (build_rope_table, build_sin_table), each value rounded once:
//   sinusoidal  [pos][D]: PE(pos, d) (sin of pair d / 2 on even d, cos on odd)
//   RoPE        [pos][D/2] words (cos, sin) of pair i < r/2, (1, 0) past the
//               rotary width (a pass-through rotation)
// Built (synchronously) when missing or too short; caller holds g_mu.
int get_table16(DeviceState& ds, const PePlan& plan, int D, int npos, hipStream_t stream,
                bool no_alloc, Table16** out) {
    const bool rope = plan.pek != atn::kPeSinusoidal;
    uint32_t base_bits;
    std::memcpy(&base_bits, &plan.base, 4);
    const auto key = std::make_tuple(rope ? 1 : 2, D, rope ? plan.rotary : D, rope ? base_bits : 0u);
    Table16& t = ds.tables16[key];
    if (t.p == nullptr || t.npos < npos) {
        if (no_alloc) return ATN_ERR_NOT_PREPARED;
        int st = refuse_if_capturing(stream);
        if (st != ATN_OK) return st;
        const int want = std::max({64, npos, t.p ? 2 * t.npos : 0});
        std::vector<float> a, b;
        std::vector<uint16_t> h((size_t)want * D);
        if (rope) {
            build_rope_table(a, b, want, plan.rotary, plan.base);
            const int nf = plan.rotary / 2;
            for (int pos = 0; pos < want; pos++)
                for (int i = 0; i < D / 2; i++) {
                    const bool on = i < nf;
                    h[(size_t)pos * D + 2 * i] = f16_bits(on ? a[(size_t)pos * nf + i] : 1.0f);
                    h[(size_t)pos * D + 2 * i + 1] = f16_bits(on ? b[(size_t)pos * nf + i] : 0.0f);
                }
        } else {
            build_sin_table(a, b, want, D);
            const int nf = (D + 1) / 2;
            for (int pos = 0; pos < want; pos++)
                for (int d = 0; d < D; d++)
                    h[(size_t)pos * D + d] =
                        f16_bits((d & 1) ? b[(size_t)pos * nf + d / 2] : a[(size_t)pos * nf + d / 2]);
        }
        if (t.p) {
            st = supersede(ds, t.p, (size_t)t.npos * D * 2, t.captured, stream, true);
            t.p = nullptr;
            t.captured = false;
            if (st != ATN_OK) return st;
        }
        ATN_HIP(hipMalloc(&t.p, h.size() * 2));
        ds.live_bytes += h.size() * 2;
        ATN_HIP(hipMemcpy(t.p, h.data(), h.size() * 2, hipMemcpyHostToDevice));
        t.npos = want;
    }
    *out = &t;
    return ATN_OK;
}

// Fills the PeSide table pointers (library tables or the caller's).
int bind_tables(const atn_pe_desc* pe, PePlan& plan, int D, int npos, hipStream_t stream,
                bool no_alloc = false) {
    if (plan.pek == atn::kPeNone) return ATN_OK;
    if (plan.caller_tables) {
        const bool rope = plan.pek != atn::kPeSinusoidal;
        for (atn::PeSide* s : {&plan.q, &plan.k}) {
            s->a = pe->table_a;
            s->b = pe->table_b;
            s->ld = rope ? plan.rotary : D;
            s->dup = 1;
        }
        return ATN_OK;
    }
    int dev;
    int st = current_device(&dev);
    if (st != ATN_OK) return st;
    std::lock_guard<std::mutex> lk(g_mu);
    Table* t = nullptr;
    st = get_table(g_dev[dev], plan, D, npos, stream, no_alloc, &t);
    if (st != ATN_OK) return st;
    if (!t->captured && is_capturing(stream)) t->captured = true;
    for (atn::PeSide* s : {&plan.q, &plan.k}) {
        s->a = t->a;
        s->b = t->b;
        s->ld = t->nfreq;
        s->dup = 0;
    }
    return ATN_OK;
}

// ---------------------------------------------------------------- streaming plan
struct StreamPlan {
    int nsplit, dchunk;
    size_t s_elems, p_elems;  // partial scores, probabilities (floats)
    size_t bytes;
};

StreamPlan stream_plan(const Shape& s) {
    StreamPlan p{};
    const int64_t tiles = s.BH * ((s.Lq + 63) / 64) * ((s.Lk + 63) / 64);
    // D-chunks until about 1024 workgroups of 64 x 64 tiles run (four per CU,
    // so that one workgroup's slice loads overlap another's MFMAs), or 512 of
    // 128 x 128 where those can run (two per CU), chunks of at least 64 dims,
    // rounded to the kernels' 32-deep slices
    const int64_t target = atn::s16_fits_128(s.Lq, s.Lk) ? 2048 : 1024;  // in 64 x 64 tiles
    int nsplit = 1;
    if (tiles < target) {
        const int64_t want = (target + tiles - 1) / tiles;
        const int64_t maxs = s.D / 64 > 1 ? s.D / 64 : 1;
        nsplit = (int)(want < maxs ? want : maxs);
    }
    int dchunk = (s.D + nsplit - 1) / nsplit;
    dchunk = (dchunk + 31) / 32 * 32;
    nsplit = (s.D + dchunk - 1) / dchunk;
    p.nsplit = nsplit;
    p.dchunk = dchunk;
    const size_t per = (size_t)s.BH * s.Lq * s.Lk;
    p.s_elems = per * nsplit;
    p.p_elems = nsplit > 1 ? per : 0;  // P aliases S when there is one split
    p.bytes = (p.s_elems + p.p_elems) * sizeof(float) + 256;
    return p;
}

int ensure_workspace(size_t bytes, hipStream_t stream, void** ws) {
    int dev;
    int st = current_device(&dev);
    if (st != ATN_OK) return st;
    std::lock_guard<std::mutex> lk(g_mu);
    DeviceState& ds = g_dev[dev];
    Workspace& w = ds.ws[stream];
    if (w.bytes < bytes) {
        st = refuse_if_capturing(stream);
        if (st != ATN_OK) return st;
        const size_t want = grown(w.bytes, bytes);
        if (w.ptr) {
            st = supersede(ds, w.ptr, w.bytes, w.captured, stream, false);
            w.ptr = nullptr;
            w.bytes = 0;
            w.captured = false;
            if (st != ATN_OK) return st;
        }
        ATN_HIP(hipMalloc(&w.ptr, want));
        ATN_HIP(hipMemset(w.ptr, 0, want));
        w.bytes = want;
        ds.live_bytes += want;
    } else if (!w.captured && is_capturing(stream)) {
        w.captured = true;
    }
    *ws = w.ptr;
    return ATN_OK;
}

// ---------------------------------------------------------------- fused plan
// Workspace layout (every path): a fixed 40 KiB sync region -- [0, 4) the
// status word, [256, 8448) one epoch word per row group of the
// single-launch kernel, [8448, 24832) two sets of 2048 per-workgroup done
// words, [32768, 40960) the XCD-local arrival counters (1 KiB per XCD) --
// then scratch.  Fixed offsets keep the epoch words and counters of one call
// from landing elsewhere when shapes change between calls.
constexpr size_t kSyncEpochOff = 256;
constexpr size_t kSyncDoneOff = 8448;
constexpr size_t kSyncXcdOff = 32768;
constexpr int kSyncMaxWorkgroups = 2048;
constexpr size_t kSyncBytes = 40960;
static_assert(kSyncXcdOff + 8 * atn::kXcdCtrWords * 4 <= kSyncBytes, "sync region");

size_t round256(size_t b) { return (b + 255) / 256 * 256; }

struct FusedPlan {
    bool ok = false;
    int MB = 0, dc = 0, nchunk = 0, lds = 0, gather1 = 0, xcd = 0, workgroups = 0;
    int per_cu = 0;  // workgroups the busiest CU runs (one round when resident)
    size_t part_words = 0, red_words = 0, bytes = 0;
};

constexpr int kFusedMaxLq = 64, kFusedMaxLk = 128;
constexpr int kLdsLimit = 160 * 1024 - 256;
constexpr int kFusedThreads = 256, kFusedMaxWords = 64;

// Words one thread of the kernel reads in each exchange step, for E scores
// per row group over n slices: the one gather (16-byte words, four entries
// of every fourth 256-entry block per thread), and the larger of the
// reduce-scatter and all-gather steps (4-byte words; their 16-byte forms
// read a quarter as many).
int gather1_words(int E, int n) { return 4 * ((E + 1023) / 1024) * n; }
int rsag_words(int E, int n) {
    const int per = (E + n - 1) / n;
    const int rs = per <= kFusedThreads ? (n + kFusedThreads / per - 1) / (kFusedThreads / per)
                                        : (per + kFusedThreads - 1) / kFusedThreads * n;
    return std::max(rs, E / kFusedThreads);
}

// Cuts each head's query rows into row groups of MB rows and D into slices
// of dc dims, one workgroup each, with the whole grid resident at once (the
// kernel's exchange waits need that: capacity is the device's CU count x
// resident workgroups per CU for the plan's LDS size; an XCD-local plan
// needs each XCD's share resident on that XCD's CUs).  Of every plan that
// fits LDS, the device and the exchange's per-thread limits, the one of least
// estimated time is taken.
FusedPlan fused_plan_uncached(int dtype, int pek, const Shape& s, bool query_device) {
    FusedPlan none;
    if (s.Lq > kFusedMaxLq || s.Lk > kFusedMaxLk || s.D % 4 != 0) return none;
    const atn_tuning& tn = tune();
    int cus = tn.model_cus > 0 ? tn.model_cus : 256;
    int xccs = tn.model_xccs > 0 ? tn.model_xccs : 8;
    int dev = 0;
    if (query_device) {
        if (hipGetDevice(&dev) != hipSuccess) return none;
        std::lock_guard<std::mutex> lk(g_mu);
        DeviceState& ds = g_dev[dev];
        if (ds.cus == 0 &&
            hipDeviceGetAttribute(&ds.cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                hipSuccess)
            return none;
        if (ds.xccs == 0 &&
            hipDeviceGetAttribute(&ds.xccs, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess)
            ds.xccs = 1;  // unknown: no XCD-local plans
        cus = ds.cus;
        xccs = ds.xccs;
    }
    // XCD-local plans assume the whole chip: 8 XCDs, each receiving every
    // eighth workgroup id and 1/8 of the CUs.  A partitioned MI355X (each
    // partition a device of 1, 2 or 4 XCDs) gets device-scope plans only.
    const bool xl_ok = xccs == 8 && cus % 8 == 0;
    auto per_cu_cap = [&](int lds) {
        std::lock_guard<std::mutex> lk(g_mu);
        int& c = g_dev[dev].fused_per_cu[std::make_pair(dtype, lds)];
        if (c == 0) c = atn::fused_small_per_cu(dtype, pek, lds);
        return c;
    };
    const int MQ = (int)(s.Lq + 15) / 16 * 16, NK = (int)(s.Lk + 31) / 32 * 32;
    const int es = dtype == ATN_DTYPE_F32 ? 4 : 2;
    // one plan: row groups of MB rows, slices of dc dims, the one-gather
    // exchange (gather = 1) or reduce-scatter + all-gather (0), exchanged at
    // device scope (xcd = 0) or inside each XCD's L2 (xcd = 1)
    auto make = [&](int MB, int dc, int gather, int xcd) {
        FusedPlan p;
        const int64_t groups = s.BH * ((s.Lq + MB - 1) / MB);
        const int64_t n = (s.D + dc - 1) / dc;
        if (groups > cus || dc > 1024 || groups * n > kSyncMaxWorkgroups) return p;
        if (n == 1 && (gather || xcd)) return p;  // a single slice has no exchange
        const int64_t gpx = (groups + 7) / 8;     // XL: row groups on the busiest XCD
        if (xcd && (!xl_ok || gpx > atn::kXcdGroupsPerXcd)) return p;
        const int lds = atn::fused_small_lds_bytes(dtype, pek, MB, (int)s.Lk, dc, (int)n);
        if (lds > kLdsLimit) return p;
        // the exchange waits need every workgroup resident; a size query (no
        // device) allows the most any plan may launch, so that the workspace
        // it reports bounds every plan the device may take
        const int per = query_device ? per_cu_cap(lds) : 8;
        if (n > 1) {
            if (per <= 0) return p;
            if (xcd ? gpx * n > (int64_t)(cus / 8) * per : groups * n > (int64_t)cus * per)
                return p;
        }
        const int E = MB * NK;
        if (n > 1) {
            if ((gather ? gather1_words(E, (int)n) : rsag_words(E, (int)n)) > kFusedMaxWords)
                return p;
            p.part_words = (size_t)(groups * n * E);
            p.red_words = gather ? 0 : (size_t)groups * E;
        }
        p.MB = MB;
        p.dc = dc;
        p.nchunk = (int)n;
        p.lds = lds;
        p.gather1 = n > 1 ? gather : 0;
        p.xcd = xcd;
        p.workgroups = (int)(groups * n);
        p.per_cu = xcd ? (int)((gpx * n + cus / 8 - 1) / (cus / 8))
                       : (int)((groups * n + cus - 1) / cus);
        p.bytes = kSyncBytes + round256(p.part_words * 4) + p.red_words * 4;
        p.ok = true;
        return p;
    };
    // Estimated time in us beyond the fixed cost.  Device-scope plans: each
    // CU's Q/K/V slice loads (0.03 us per KiB), the slices (0.02 us each),
    // reduce-scatter's second round trip (1 us), each CU's exchange reads
    // (0.04 us per KiB) and the workgroup count (0.358 us per CU's worth).
    // XCD-local plans: 2 us less, reduce-scatter's second step 2.5 us, and
    // exchange reads from L2 no cost of their own at this resolution; their
    // XCDs also fetch whole heads' K and V (each XCD holds a block of row
    // groups), where device-scope plans spread every head over all 8: the
    // extra bytes per XCD cost about 1 us per MB.  The coefficients were
    // chosen against a sweep that timed every plan of 15 fp32/bf16 shapes
    // (269 plans, B*H 1-16, Lq 16-64, Lk 16-128, D 512-8192): on it they pick
    // the fastest measured plan of every shape, and fitted on 14 shapes they
    // lose 0.6 us in total on the 15 held out in turn.
    const double kv_head = 2.0 * (double)s.Lk * (double)s.D * es;
    auto cost = [&](const FusedPlan& p) {
        const double per_cu = (double)p.per_cu;
        const double kib = (double)(std::min(p.MB, MQ) + 2 * NK) * p.dc * es / 1024.0;
        const double E = (double)p.MB * NK;
        const double xkib = p.nchunk == 1 ? 0.0 : (p.gather1 ? E * p.nchunk : 2.0 * E) * 4 / 1024.0;
        if (p.xcd) {
            const int QB = (int)((s.Lq + p.MB - 1) / p.MB);
            const int64_t G = s.BH * QB, gpx = (G + 7) / 8;
            const double heads_x = (double)std::max<int64_t>(1, (gpx + QB - 1) / QB);
            const double kv_extra = std::max(0.0, heads_x * kv_head - (double)s.BH * kv_head / 8.0);
            return 0.03 * kib * per_cu + 0.02 * p.nchunk + (!p.gather1 ? 2.5 : 0.0) +
                   0.358 * p.workgroups / cus - 2.0 + kv_extra * 1e-6;
        }
        return 0.03 * kib * per_cu + 0.02 * p.nchunk + (p.nchunk > 1 && !p.gather1 ? 1.0 : 0.0) +
               0.04 * xkib * per_cu + 0.358 * p.workgroups / cus;
    };
    // overrides (atn_tuning): row group size, slice width, exchange, scope
    const int force_rows = tn.fused_rows > 0 ? tn.fused_rows : 0;
    const int force_dc = tn.fused_dc >= 32 && tn.fused_dc % 32 == 0 ? tn.fused_dc : 0;
    const int force_x = tn.fused_exchange == 1 ? 1 : (tn.fused_exchange == 2 ? 0 : -1);
    const int force_xcd = tn.fused_xcd == 1 ? 1 : (tn.fused_xcd == 2 ? 0 : -1);
    const bool forced = force_rows > 0 || force_dc > 0 || force_x >= 0 || force_xcd >= 0;
    // candidates: row groups of 64, 32 or 16 rows (48: the whole padded head
    // of 33-48 rows), slices of 32-512 dims and the width that gives one
    // workgroup per CU
    FusedPlan best, best_forced;
    size_t max_bytes = 0;
    for (int MB : {64, 48, 32, 16}) {
        if (MB > MQ || (MB == 48 && MQ != 48)) continue;
        const int64_t groups = s.BH * ((s.Lq + MB - 1) / MB);
        if (groups > cus) continue;
        const int64_t per_group = cus / groups;
        const int natural = (int)(((s.D + per_group - 1) / per_group + 31) / 32 * 32);
        const int whole = (int)((s.D + 31) / 32 * 32);
        for (int dc : {32, 64, 128, 256, 512, natural}) {
            dc = std::min(dc, whole);
            for (int gather : {1, 0})
                for (int xcd : {0, 1}) {
                    const FusedPlan p = make(MB, dc, gather, xcd);
                    if (!p.ok) continue;
                    max_bytes = std::max(max_bytes, p.bytes);
                    if (!best.ok || cost(p) < cost(best)) best = p;
                    if (forced && (force_rows == 0 || p.MB == force_rows) &&
                        (force_dc == 0 || p.dc == force_dc) &&
                        (force_x < 0 || p.nchunk == 1 || p.gather1 == force_x) &&
                        (force_xcd < 0 || p.nchunk == 1 || p.xcd == force_xcd) &&
                        (!best_forced.ok || cost(p) < cost(best_forced)))
                        best_forced = p;
                }
        }
    }
    FusedPlan p = best_forced.ok ? best_forced : best;
    if (!query_device && p.ok) p.bytes = max_bytes;
    return p;
}

// Plans are cached per (device, dtype, encoding, shape), the size query's
// under device -1; atn_set_tuning_ex drops the cache.
std::map<std::tuple<int, int, int, int64_t, int64_t, int64_t, int64_t>, FusedPlan> g_fused_plans;

FusedPlan fused_plan(int dtype, int pek, const Shape& s, bool query_device) {
    int dev = -1;
    if (query_device && hipGetDevice(&dev) != hipSuccess) return FusedPlan{};
    const auto key = std::make_tuple(dev, dtype, pek, (int64_t)s.BH, (int64_t)s.Lq,
                                     (int64_t)s.Lk, (int64_t)s.D);
    {
        std::lock_guard<std::mutex> lk(g_mu);
        const auto it = g_fused_plans.find(key);
        if (it != g_fused_plans.end()) return it->second;
    }
    const FusedPlan p = fused_plan_uncached(dtype, pek, s, query_device);
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_fused_plans.size() >= 4096) g_fused_plans.clear();
    g_fused_plans.emplace(key, p);
    return p;
}

// ---------------------------------------------------------------- gemm plan
// bf16 shapes outside the single-launch kernel's window: two MFMA GEMMs
// around an exact row softmax.  Workspace after the sync region: encoded Q
// and K (fp16 with per-row scales, when a positional encoding is on), E =
// exp(S - tile row max) (fp16, rows padded to ldE = Lk rounded up to 8 keys),
// per-(row, 256-key tile) max, sum and softmax factor (fp32).
struct GemmPlan {
    bool ok = false, encoded = false;
    int benc = 0;     // fused K encoding (atn::kGemmEnc*), 0 = K~ from k_encode_f16
    int ldE = 0;      // E row stride (elements)
    int tiles_k = 0;  // 256-key tiles per score row
    size_t q_off = 0, k_off = 0, qs_off = 0, ks_off = 0, e_off = 0, m_off = 0, l_off = 0,
           g_off = 0, bytes = 0;
};

GemmPlan gemm_plan(int dtype, const Shape& s, const PePlan& plan) {
    GemmPlan p;
    if (dtype != ATN_DTYPE_BF16 || s.D % 8 != 0) return p;
    p.ldE = (int)((s.Lk + 7) / 8 * 8);
    // the GEMM kernels address one head's matrix with 32-bit element offsets
    const int64_t lim = (int64_t)1 << 31;
    if ((int64_t)s.Lq * s.D >= lim || (int64_t)s.Lk * s.D >= lim || (int64_t)s.Lq * p.ldE >= lim)
        return p;
    size_t off = kSyncBytes;
    auto take = [&](size_t b) { size_t o = off; off += round256(b); return o; };
    // with a positional encoding the query side is re-encoded as scaled fp16,
    // and so is the key side unless its encoding runs inside the QK^T GEMM
    // (k_gemm_qk_enc: fp16 tables, no K~ pass).  That takes an even number of
    // 64-deep K steps, the library's tables, rotate-half over all of D, and
    // at most four 256-row query tiles: every query tile's workgroups encode
    // their K tiles again, so the in-GEMM encoding grows with Lq while the
    // K~ pass does not (config 4, four query tiles: 724 us fused against
    // 545 + 198 us, so the break-even is near 1100 rows; config 5, one query
    // tile: 112 us against 143 + 110 us).
    // atn_tuning.gemm_fused_k turns it off (2) or on wherever it can run (1).
    p.encoded = plan.pek != atn::kPeNone;
    const int fk = tune().gemm_fused_k;
    if (p.encoded && s.D % 128 == 0 && !plan.caller_tables && fk != 2 &&
        (fk == 1 || (s.Lq + 255) / 256 <= 4)) {
        if (!plan.k.on)
            p.benc = atn::kGemmEncRaw;
        else if (plan.pek == atn::kPeSinusoidal)
            p.benc = atn::kGemmEncSin;
        else if (plan.pek == atn::kPeRopeInterleaved)
            p.benc = atn::kGemmEncRope;
        else if (plan.pek == atn::kPeRopeHalf && plan.rotary == s.D)
            p.benc = atn::kGemmEncRopeHalf;
    }
    if (p.encoded) {
        p.q_off = take((size_t)s.BH * s.Lq * s.D * 2);
        p.qs_off = take((size_t)s.BH * s.Lq * 4);
        if (p.benc == 0) {
            p.k_off = take((size_t)s.BH * s.Lk * s.D * 2);
            p.ks_off = take((size_t)s.BH * s.Lk * 4);
        }
    }
    p.tiles_k = (int)((s.Lk + 255) / 256);
    const size_t stats = (size_t)s.BH * s.Lq * p.tiles_k * 4;
    p.e_off = take((size_t)s.BH * s.Lq * p.ldE * 2);
    p.m_off = take(stats);
    p.l_off = take(stats);
    p.g_off = take(stats);
    p.bytes = off;
    p.ok = true;
    return p;
}

// ---------------------------------------------------------------- core
// Scratch the library may use for one call before splitting it: the
// caller's workspace size, the allocation-free array, or this cap for the
// library's own workspace (atn_tuning.workspace_cap_mib overrides it).
size_t library_cap() {
    const int mib = tune().workspace_cap_mib;
    return mib > 0 ? (size_t)mib << 20 : (size_t)1 << 30;
}

// The flash kernel takes fp32 and bf16 calls with head_d <= 256 (128 with
// an encoding), head_d % 4 == 0 and 16-byte aligned bases (checked by the
// caller), whose per-head Q and K/V byte offsets fit 32 bits.  bf16 calls
// with an encoding past head_d 128 therefore take the GEMM path.  Without
// one the flash kernel's bf16 products run on the raw bits, and at head_d
// 256 it ties or beats the GEMM path (same box, flash at head_d 252 against
// the GEMM path at 256: (4,32,512,512) 64.0 / 64.4 us, (2,16,1024,1024)
// 54.6 / 66.9 us, (1,8,4096,4096) 165 / 315 us).
bool flash_ok(int dtype, const Shape& s, const PePlan& plan) {
    const int64_t lim = (int64_t)1 << 31;
    const int64_t es = dtype == ATN_DTYPE_F32 ? 4 : 2;
    return !plan.no_flash && atn::flash_supported(dtype, plan.pek, s.D) &&
           (int64_t)s.Lq * s.D * es < lim && (int64_t)s.Lk * s.D * es < lim;
}

// The flash kernel's workgroup form (atn_tuning.flash_form forces one).
// 8 waves of 32 query rows (32 x 32 MFMA tiles: each wave reads a K/V tile
// from LDS once per 32 rows, and each tile is converted once per 256 rows)
// when head_d <= 128 and the grid of 256-row blocks gives every CU a
// workgroup; else 8 waves of 16 rows (twice the workgroups).  Measured
// with interleaved rounds on 14 shapes: the reference's (4,32,512,512,128)
// 70.6 -> 62.9 us, RoPE there 108 -> 86 us; below a workgroup per CU the
// 32-row form loses (up to 1.6x at (1,4,2048,2048,128)).  Up to 64 query
// rows, 4 waves of 16 rows (64-row blocks: no wave of padding rows; with key
// splits, same box: (1,32,16,4096,128) bf16 33.2 -> 29.6 us, (1,8,64,4096,
// 128) fp32 35.7 -> 33.8 us).  From 4096 keys on, the 32-row form even below
// a workgroup per CU (its key splits then fill the grid): each K/V tile read
// and encoded once per 256 rows outweighs the splits' merge there (same box:
// bf16 (1,8,4096,4096,128) 102 -> 91 us, (1,2,16384,16384,128) 346 -> 280 us,
// RoPE rotate-half 173 -> 128 us, sinusoidal (1,4,8192,8192,128) 338 -> 216
// us, fp32 (1,4,8192,8192,128) 432 -> 395 us, fp32 (1,8,4096,4096,64) 131
// -> 123 us; at 1024 keys the 16-row form stays ahead: 33 against 43 us at
// (2,16,1024,1024,128)).
int flash_form(const Shape& s, int dev) {
    const int forced = tune().flash_form;
    if (forced >= atn::kFlashForm4x16 && forced <= atn::kFlashForm8x32) return forced;
    if (s.D > 128) return atn::kFlashForm8x16;
    if (s.Lq <= 64) return atn::kFlashForm4x16;
    int cus = 0;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        DeviceState& ds = g_dev[dev];
        if (ds.cus == 0 &&
            hipDeviceGetAttribute(&ds.cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                hipSuccess)
            ds.cus = 0;
        cus = ds.cus > 0 ? ds.cus : 256;
    }
    if (s.BH * ((s.Lq + 255) / 256) >= (int64_t)cus) return atn::kFlashForm8x32;
    return s.Lk >= 4096 ? atn::kFlashForm8x32 : atn::kFlashForm8x16;
}

// Query rows per workgroup of a flash form.
int flash_rows(int form, int D) {
    if (D > 128) form = atn::kFlashForm8x16;
    return form == atn::kFlashForm4x16 ? 64 : (form == atn::kFlashForm8x32 ? 256 : 128);
}

// Key splits of the flash kernel.  A workgroup walks all keys of its query
// block, so a grid of few (head, query block) pairs leaves CUs idle (64
// workgroups at (1,4,2048,2048,128), 32 for 16 queries against 4096 keys at
// 32 heads).  Such calls split the keys into parts of whole 64-key chunks,
// two at least, so that the grid reaches about kFlashSplitTarget workgroups;
// each part writes its normalized output and statistics (fp32) and a second
// kernel merges them.  Decided from the shape alone (plus
// atn_tuning.flash_split), so the workspace queries need no device.
struct FlashSplit {
    int nsplit = 1, kchunk = 0;
    size_t bytes = 0;  // scratch of the parts
};
constexpr int kFlashSplitTarget = 256, kFlashSplitBelow = 128, kFlashSplitMax = 32;

FlashSplit flash_split(const Shape& s, int rows) {
    FlashSplit f;
    const int forced = tune().flash_split;
    if (forced == 1) return f;
    const int64_t grid = s.BH * ((s.Lq + rows - 1) / rows);
    const int chunks = (s.Lk + 63) / 64;
    int64_t n;
    if (forced >= 2) {
        n = std::min<int64_t>(forced, chunks);
    } else {
        if (grid > kFlashSplitBelow) return f;
        n = std::min<int64_t>({(kFlashSplitTarget + grid - 1) / grid, chunks / 2, kFlashSplitMax});
    }
    if (n < 2) return f;
    f.kchunk = (int)((chunks + n - 1) / n) * 64;
    f.nsplit = (s.Lk + f.kchunk - 1) / f.kchunk;
    if (f.nsplit < 2) return FlashSplit{};
    f.bytes = (size_t)f.nsplit * s.BH * s.Lq * (s.D + 4) * 4;
    return f;
}

// The most scratch any flash form's split of this shape takes.
size_t flash_split_bound(const Shape& s) {
    size_t b = 0;
    for (int rows : {64, 128, 256}) b = std::max(b, flash_split(s, rows).bytes);
    return b;
}

// Scratch bytes of the path a call of shape s takes: fused (when planned and
// vector-aligned), else GEMM (when planned and 16-byte aligned), else the
// split-D pipeline.  vec / a16: the alignment of the call's pointers; pass
// -1 for "unknown" and get the largest of the candidate paths instead.
size_t path_need(int dtype, const Shape& s, const PePlan& plan, bool query_device, int vec,
                 int a16) {
    const FusedPlan fp = plan.no_fused ? FusedPlan{} : fused_plan(dtype, plan.pek, s, query_device);
    const GemmPlan gp = gemm_plan(dtype, s, plan);
    const size_t split = kSyncBytes + stream_plan(s).bytes;
    if (vec < 0 || a16 < 0)
        return std::max({fp.ok ? fp.bytes : (size_t)0, gp.ok ? gp.bytes : (size_t)0, split,
                         flash_ok(dtype, s, plan) ? kSyncBytes + flash_split_bound(s)
                                                  : (size_t)0});
    if (fp.ok && vec) return fp.bytes;
    if (a16 && flash_ok(dtype, s, plan))  // the flash kernel: only its key splits' parts
        return kSyncBytes + flash_split_bound(s);
    if (gp.ok && a16) return gp.bytes;
    return split;
}

// How a call too large for its scratch is split: chunks of `heads`
// consecutive (batch, head) pairs, or, when one head is still too large,
// chunks of `rows` query rows of one head (K and V whole).  Each chunk is an
// independent attention call: rows depend only on their own query row and
// all keys.
struct Chunking {
    int heads = 0, rows = 0;  // heads == 0: no chunk fits
    size_t need = 0;          // largest chunk's scratch
};

Chunking plan_chunks(int dtype, const Shape& s, const PePlan& plan, size_t cap,
                     bool query_device, int vec, int a16) {
    auto need_of = [&](int h, int rows) {
        Shape c;
        check_shape(1, h, rows, s.Lk, s.D, &c);
        return path_need(dtype, c, plan, query_device, vec, a16);
    };
    Chunking ch;
    int h = (int)s.BH;
    size_t n = need_of(h, s.Lq);
    while (h > 1 && n > cap) {
        h = (h + 1) / 2;
        n = need_of(h, s.Lq);
    }
    if (n <= cap) {
        ch.heads = h;
        ch.rows = s.Lq;
        ch.need = n;
        return ch;
    }
    int r = s.Lq;
    while (r > 1 && n > cap) {
        r = (r + 1) / 2;
        n = need_of(1, r);
    }
    if (n <= cap) {
        ch.heads = 1;
        ch.rows = r;
        ch.need = n;
    }
    return ch;
}

// One call of the chosen path on (a chunk of) the job, tables already
// bound; plan.q's tables start at the chunk's first query position.
int attention_run(int dtype, const void* Q, const void* K, const void* V, void* out,
                  const Shape& s, const PePlan& plan, int dev, void* workspace,
                  size_t workspace_bytes, hipStream_t stream, bool no_alloc) {
    const int Lq = s.Lq, Lk = s.Lk, D = s.D;
    int st = ATN_OK;
    const GemmPlan gp = gemm_plan(dtype, s, plan);
    const StreamPlan sp = stream_plan(s);
    // the device's own capacity decides between the single-launch kernel
    // and the three-kernel pipeline
    const FusedPlan fd = plan.no_fused ? FusedPlan{} : fused_plan(dtype, plan.pek, s, true);
    const size_t va = dtype == ATN_DTYPE_F32 ? 16 : 8;
    const int vec_qk = (D % 4 == 0) && aligned(Q, va) && aligned(K, va);
    const int vec_vo = (D % 4 == 0) && aligned(V, va) && aligned(out, va);
    const bool use_fused = fd.ok && vec_qk && vec_vo;
    const bool a16 = aligned(Q, 16) && aligned(K, 16) && aligned(V, 16) && aligned(out, 16);
    const bool use_flash = !use_fused && a16 && flash_ok(dtype, s, plan);
    const bool use_gemm = !use_fused && !use_flash && gp.ok && aligned(Q, 16) && aligned(K, 16) &&
                          aligned(V, 16) && aligned(out, 16);
    const int fform = use_flash ? flash_form(s, dev) : 0;
    const FlashSplit fs = use_flash ? flash_split(s, flash_rows(fform, D)) : FlashSplit{};
    const size_t need =
        use_fused ? fd.bytes
                  : (use_flash ? kSyncBytes + fs.bytes
                               : (use_gemm ? gp.bytes : kSyncBytes + sp.bytes));
    void* ws = workspace;
    if (no_alloc) {
        if (need > atn::kNoAllocScratchBytes) return ATN_ERR_SCRATCH_LIMIT;
        if (!atn::noalloc_ready(dev)) {
            // set-up (symbol address, sync region cleared) runs once per
            // device, outside capture
            st = refuse_if_capturing(stream);
            if (st != ATN_OK) return st;
        }
        ATN_HIP(atn::noalloc_scratch(dev, kSyncBytes, stream, &ws));
    } else if (ws == nullptr) {
        st = ensure_workspace(need, stream, &ws);
        if (st != ATN_OK) return st;
    } else if (workspace_bytes < need) {
        return ATN_ERR_WORKSPACE;
    }
    int* status = reinterpret_cast<int*>(ws);
    const float scale = 1.0f / sqrtf((float)D);  // final/attention.cu:206

    float* scratch = reinterpret_cast<float*>((char*)ws + kSyncBytes);
    if (use_gemm) {
        char* w = static_cast<char*>(ws);
        const uint16_t* qe = static_cast<const uint16_t*>(Q);
        const uint16_t* ke = static_cast<const uint16_t*>(K);
        uint16_t* E = reinterpret_cast<uint16_t*>(w + gp.e_off);
        float* st_m = reinterpret_cast<float*>(w + gp.m_off);
        float* st_l = reinterpret_cast<float*>(w + gp.l_off);
        float* ga = reinterpret_cast<float*>(w + gp.g_off);
        if (gp.encoded) {
            uint16_t* qd = reinterpret_cast<uint16_t*>(w + gp.q_off);
            uint16_t* kd = reinterpret_cast<uint16_t*>(w + gp.k_off);
            float* qs = reinterpret_cast<float*>(w + gp.qs_off);
            float* ks = reinterpret_cast<float*>(w + gp.ks_off);
            ATN_HIP(atn::launch_encode_f16(plan.q.on ? plan.pek : atn::kPeNone, qe, qd, qs,
                                           (long)(s.BH * Lq), Lq, D, plan.q, stream));
            if (gp.benc != 0) {
                // K encoded inside the QK^T GEMM
                const uint16_t* tab = nullptr;
                int tab_rows = 0;
                if (gp.benc != atn::kGemmEncRaw) {
                    std::lock_guard<std::mutex> lk(g_mu);
                    Table16* t16 = nullptr;
                    st = get_table16(g_dev[dev], plan, D, Lq > Lk ? Lq : Lk, stream, no_alloc,
                                     &t16);
                    if (st != ATN_OK) return st;
                    if (!t16->captured && is_capturing(stream)) t16->captured = true;
                    tab = t16->p;
                    tab_rows = t16->npos;
                }
                ATN_HIP(atn::launch_gemm_qk_enc(gp.benc, qd, ke, qs, tab, tab_rows, E, gp.ldE, st_m,
                                                st_l, (int)s.BH, Lq, Lk, D, scale, stream));
            } else {
                ATN_HIP(atn::launch_encode_f16(plan.k.on ? plan.pek : atn::kPeNone, ke, kd, ks,
                                               (long)(s.BH * Lk), Lk, D, plan.k, stream));
                ATN_HIP(atn::launch_gemm_qk(1, qd, kd, qs, ks, E, gp.ldE, st_m, st_l, (int)s.BH, Lq,
                                            Lk, D, scale, stream));
            }
        } else {
            ATN_HIP(atn::launch_gemm_qk(0, qe, ke, nullptr, nullptr, E, gp.ldE, st_m, st_l,
                                        (int)s.BH, Lq, Lk, D, scale, stream));
        }
        ATN_HIP(atn::launch_gemm_pv(E, gp.ldE, st_m, st_l, ga, static_cast<const uint16_t*>(V),
                                    static_cast<uint16_t*>(out), (int)s.BH, Lq, Lk, D, stream));
        return ATN_OK;
    }
    if (use_fused) {
        unsigned* epochs = reinterpret_cast<unsigned*>((char*)ws + kSyncEpochOff);
        float* part = reinterpret_cast<float*>((char*)ws + kSyncBytes);
        float* red = reinterpret_cast<float*>((char*)ws + kSyncBytes + round256(fd.part_words * 4));
        unsigned* done = reinterpret_cast<unsigned*>((char*)ws + kSyncDoneOff);
        unsigned* xctr = reinterpret_cast<unsigned*>((char*)ws + kSyncXcdOff);
        if (tune().preset_status) {
            // test control (atn_tuning.preset_status): the status word set as
            // a timed-out call leaves it, so that every workgroup takes the
            // fail-closed exit (no wait is entered); never recorded into a
            // graph
            if (is_capturing(stream)) return ATN_ERR_CAPTURE;
            ATN_HIP(hipMemsetAsync(status, 0x01, 1, stream));
        }
        ATN_HIP(atn::launch_fused_small(dtype, plan.pek, Q, K, V, out, part, red, epochs, done,
                                        status, xctr, (int)s.BH, Lq, Lk, D, fd.MB, fd.dc,
                                        fd.nchunk, fd.gather1, fd.xcd, scale, plan.q, plan.k,
                                        stream));
        return ATN_OK;
    }
    if (use_flash) {
        ATN_HIP(atn::launch_flash(dtype, plan.pek, fform, Q, K, V, out, (int)s.BH, Lq, Lk, D,
                                  scale, plan.q, plan.k, fs.nsplit, fs.kchunk, scratch, stream));
        return ATN_OK;
    }
    float* S = scratch;
    float* P = sp.nsplit > 1 ? S + sp.s_elems : S;
    ATN_HIP(atn::launch_qk_partial(dtype, plan.pek, Q, K, S, (int)s.BH, Lq, Lk, D, sp.dchunk,
                                   sp.nsplit, plan.q, plan.k, vec_qk, stream));
    ATN_HIP(atn::launch_softmax(S, P, s.BH * Lq, Lk, sp.nsplit, (size_t)s.BH * Lq * Lk, scale,
                                stream));
    ATN_HIP(atn::launch_pv(dtype, P, V, out, (int)s.BH, Lq, Lk, D, vec_vo, stream));
    return ATN_OK;
}


// no_alloc: the allocation-free form -- scratch is the device's static
// array, and a call that would need a library allocation (tables not yet
// built) is refused.  A call whose scratch would exceed the cap (the
// caller's workspace, the static array, or library_cap()) is run in chunks
// of heads or query rows that fit it.
int attention_core(int dtype, const void* Q, const void* K, const void* V, void* out, int B,
                   int H, int Lq, int Lk, int D, const atn_pe_desc* pe, void* workspace,
                   size_t workspace_bytes, hipStream_t stream, bool no_alloc = false,
                   bool no_fused = false) {
    if (dtype != ATN_DTYPE_F32 && dtype != ATN_DTYPE_BF16) return ATN_ERR_BAD_ARGUMENT;
    if (!Q || !K || !V || !out) return ATN_ERR_NULL_POINTER;
    Shape s;
    int st = check_shape(B, H, Lq, Lk, D, &s);
    if (st != ATN_OK) return st;
    const size_t es = elem_size(dtype);
    for (const void* p : {Q, K, V, (const void*)out})
        if (!aligned(p, es)) return ATN_ERR_MISALIGNED;
    const int64_t qb = s.nq * (int64_t)es, kb = s.nk * (int64_t)es;
    if (overlaps(out, qb, Q, qb) || overlaps(out, qb, K, kb) || overlaps(out, qb, V, kb))
        return ATN_ERR_ALIASING;
    PePlan plan;
    st = check_pe(pe, D, &plan);
    if (st != ATN_OK) return st;
    plan.no_fused = no_fused || tune().no_fused != 0;
    plan.no_flash = tune().no_flash != 0;
    // every path needs at least the sync region; the path-specific size is
    // checked once the device has chosen the path
    if (workspace != nullptr && workspace_bytes < kSyncBytes) return ATN_ERR_WORKSPACE;
    {
        const StreamPlan sp = stream_plan(s);
        const int64_t tiles = s.BH * ((Lq + 63) / 64) * ((Lk + 63) / 64) * sp.nsplit;
        const int64_t pv_tiles = s.BH * ((Lq + 63) / 64) * ((D + 63) / 64);
        if (tiles > (1LL << 24) || pv_tiles > (1LL << 24)) return ATN_ERR_SIZE_OVERFLOW;
    }

    int dev;
    st = current_device(&dev);
    if (st != ATN_OK) return st;
    st = bind_tables(pe, plan, D, Lq > Lk ? Lq : Lk, stream, no_alloc);
    if (st != ATN_OK) return st;

    const size_t cap = no_alloc ? atn::kNoAllocScratchBytes
                                : (workspace != nullptr ? workspace_bytes : library_cap());
    // chunk pointers keep the base alignment when a row is a multiple of 16
    // bytes; otherwise plan for the largest path
    const size_t va = dtype == ATN_DTYPE_F32 ? 16 : 8;
    const bool rows16 = ((size_t)D * es) % 16 == 0;
    const int vec = rows16 ? ((D % 4 == 0) && aligned(Q, va) && aligned(K, va) &&
                              aligned(V, va) && aligned(out, va))
                           : -1;
    const int a16 = rows16 ? (aligned(Q, 16) && aligned(K, 16) && aligned(V, 16) &&
                              aligned(out, 16))
                           : -1;
    if (path_need(dtype, s, plan, true, vec, a16) <= cap)
        return attention_run(dtype, Q, K, V, out, s, plan, dev, workspace, workspace_bytes,
                             stream, no_alloc);
    const Chunking ch = plan_chunks(dtype, s, plan, cap, true, vec, a16);
    if (ch.heads == 0) return no_alloc ? ATN_ERR_SCRATCH_LIMIT : ATN_ERR_WORKSPACE;
    const char* q8 = static_cast<const char*>(Q);
    const char* k8 = static_cast<const char*>(K);
    const char* v8 = static_cast<const char*>(V);
    char* o8 = static_cast<char*>(out);
    const size_t qrow = (size_t)D * es;
    for (int64_t bh0 = 0; bh0 < s.BH; bh0 += ch.heads) {
        const int h = (int)std::min<int64_t>(ch.heads, s.BH - bh0);
        for (int r0 = 0; r0 < Lq; r0 += ch.rows) {
            const int rows = std::min(ch.rows, Lq - r0);
            Shape c;
            check_shape(1, h, rows, Lk, D, &c);
            PePlan pc = plan;
            if (r0 > 0 && pc.pek != atn::kPeNone) {
                // positions of this chunk's query rows start at r0
                pc.q.a += (size_t)r0 * pc.q.ld;
                pc.q.b += (size_t)r0 * pc.q.ld;
            }
            const size_t qoff = ((size_t)bh0 * Lq + r0) * qrow, koff = (size_t)bh0 * Lk * qrow;
            st = attention_run(dtype, q8 + qoff, k8 + koff, v8 + koff, o8 + qoff, c, pc, dev,
                               workspace, workspace_bytes, stream, no_alloc);
            if (st != ATN_OK) return st;
        }
    }
    return ATN_OK;
}

int pe_apply_core(int dtype, const void* in, void* out, long n_rows, int seq_len, int D,
                  const atn_pe_desc* pe, hipStream_t stream) {
    if (dtype != ATN_DTYPE_F32 && dtype != ATN_DTYPE_BF16) return ATN_ERR_BAD_ARGUMENT;
    if (!in || !out || !pe) return ATN_ERR_NULL_POINTER;
    if (n_rows < 1 || seq_len < 1 || D < 1) return ATN_ERR_BAD_DIMENSION;
    int64_t n;
    if (!mul_ok(n_rows, D, &n) || n > INT64_MAX / 8) return ATN_ERR_SIZE_OVERFLOW;
    const size_t es = elem_size(dtype);
    if (!aligned(in, es) || !aligned(out, es)) return ATN_ERR_MISALIGNED;
    if (in != out && overlaps(in, n * (int64_t)es, out, n * (int64_t)es))
        return ATN_ERR_ALIASING;
    atn_pe_desc d = *pe;
    d.apply_q = d.apply_k = 1;
    PePlan plan;
    int st = check_pe(&d, D, &plan);
    if (st != ATN_OK) return st;
    if (plan.pek == atn::kPeNone) return ATN_ERR_BAD_ARGUMENT;
    int dev;
    st = current_device(&dev);
    if (st != ATN_OK) return st;
    st = bind_tables(&d, plan, D, seq_len, stream);
    if (st != ATN_OK) return st;
    const size_t va = dtype == ATN_DTYPE_F32 ? 16 : 8;
    const int vec = (D % 4 == 0) && aligned(in, va) && aligned(out, va);
    ATN_HIP(atn::launch_pe_apply(dtype, plan.pek, in, out, n_rows, seq_len, D, plan.q, vec,
                                 stream));
    return ATN_OK;
}

// ---------------------------------------------------------------- drop-in helpers
[[noreturn]] void die(int status, const char* where) {
    std::fprintf(stderr, "attn_mi355x error %d (%s) at %s", status, atn_status_string(status),
                 where);
    if (status == ATN_ERR_HIP || status == ATN_ERR_NO_DEVICE)
        std::fprintf(stderr, " [hip %d: %s]", g_last_hip_error,
                     hipGetErrorString((hipError_t)g_last_hip_error));
    std::fprintf(stderr, "\n");
    std::exit(EXIT_FAILURE);
}

// After the stream has drained: reads the status word of a workspace (the
// library's own for `stream` when ws == NULL).  An exchange timeout is
// reported once; the status word is cleared and every epoch word moves one
// step on, past the epoch whose exchange words the failed call may have
// left behind, which re-enables the single-launch kernel (XCD-local
// counters stay consistent by themselves).
int workspace_status(void* ws, hipStream_t stream) {
    int dev;
    int st = current_device(&dev);
    if (st != ATN_OK) return st;
    if (ws == nullptr) {
        // the stream's library workspace, then the device's allocation-free
        // scratch (once it is set up)
        void* lib_ws = nullptr;
        {
            std::lock_guard<std::mutex> lk(g_mu);
            auto& m = g_dev[dev].ws;
            auto it = m.find(stream);
            if (it != m.end()) lib_ws = it->second.ptr;
        }
        const int a = lib_ws != nullptr ? workspace_status(lib_ws, stream) : ATN_OK;
        int b = ATN_OK;
        if (atn::noalloc_ready(dev)) {
            void* sc = nullptr;
            ATN_HIP(atn::noalloc_scratch(dev, kSyncBytes, stream, &sc));
            b = workspace_status(sc, stream);
        }
        return a != ATN_OK ? a : b;
    }
    int word = 0;
    ATN_HIP(hipMemcpy(&word, ws, sizeof(int), hipMemcpyDeviceToHost));
    if (word == 0) return ATN_OK;
    std::vector<unsigned> epochs(kSyncMaxWorkgroups);
    char* e_dev = static_cast<char*>(ws) + kSyncEpochOff;
    ATN_HIP(hipMemcpy(epochs.data(), e_dev, epochs.size() * 4, hipMemcpyDeviceToHost));
    for (unsigned& e : epochs) e += 1u;
    ATN_HIP(hipMemcpy(e_dev, epochs.data(), epochs.size() * 4, hipMemcpyHostToDevice));
    ATN_HIP(hipMemset(ws, 0, sizeof(int)));
    return ATN_ERR_DEVICE_TIMEOUT;
}

// Completion of a synchronous drop-in call (enqueued on the null stream):
// the status word of the null stream's library workspace, the only
// workspace a drop-in uses, is copied into a pinned host word behind the
// call, so the one device synchronization covers the call and its status
// check.  A set word runs the recovery of workspace_status() and returns
// ATN_ERR_DEVICE_TIMEOUT; any other failure ends the process (the
// reference's CUDA_CHECK, final/attention.cu:12-21).  The allocation-free
// scratch is not looked at: its status belongs to the noalloc callers, who
// query it with atn_sync_status_ex.
int finish_sync(int status, const char* where) {
    if (status != ATN_OK) die(status, where);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        g_last_hip_error = (int)e;
        die(ATN_ERR_HIP, where);
    }
    int dev;
    int st = current_device(&dev);
    if (st != ATN_OK) die(st, where);
    void* lib_ws = nullptr;
    int* host = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        DeviceState& ds = g_dev[dev];
        auto it = ds.ws.find(nullptr);
        if (it != ds.ws.end()) lib_ws = it->second.ptr;
        if (ds.status_host == nullptr) {
            void* p = nullptr;
            if (hipHostMalloc(&p, 2 * sizeof(int), hipHostMallocDefault) == hipSuccess)
                ds.status_host = static_cast<int*>(p);
        }
        host = ds.status_host;
    }
    bool copied = host != nullptr;
    if (copied && lib_ws != nullptr)
        copied = hipMemcpyAsync(&host[0], lib_ws, sizeof(int), hipMemcpyDeviceToHost, nullptr) ==
                 hipSuccess;
    e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        g_last_hip_error = (int)e;
        die(ATN_ERR_HIP, where);
    }
    // without the pinned word (or after a failed copy), the blocking read
    if (lib_ws != nullptr && (!copied || host[0] != 0)) {
        const int ws = workspace_status(lib_ws, nullptr);
        if (ws != ATN_OK && ws != ATN_ERR_DEVICE_TIMEOUT) die(ws, where);
        return ws;
    }
    return ATN_OK;
}

void sync_or_die(int status, const char* where) {
    const int st = finish_sync(status, where);
    if (st != ATN_OK) die(st, where);
}

// A synchronous attention call (the drop-ins).  When the single-launch
// kernel's exchange timed out -- its waits need the whole grid resident, and
// work elsewhere on the device held CUs the grid needed -- the workspace has
// been recovered and the call runs once more without that kernel, on kernels
// that wait on no other workgroup; a second failure ends the process.
void dropin_attention(const char* where, int dtype, const void* Q, const void* K, const void* V,
                      void* out, int B, int H, int Lq, int Lk, int D, const atn_pe_desc* pe) {
    if (finish_sync(attention_core(dtype, Q, K, V, out, B, H, Lq, Lk, D, pe, nullptr, 0, nullptr),
                    where) == ATN_OK)
        return;
    g_reruns.fetch_add(1, std::memory_order_relaxed);
    std::fprintf(stderr,
                 "attn_mi355x: %s: the single-launch kernel's wait timed out; running the call "
                 "again without it\n",
                 where);
    sync_or_die(attention_core(dtype, Q, K, V, out, B, H, Lq, Lk, D, pe, nullptr, 0, nullptr,
                               false, true),
                where);
}

atn_pe_desc rope_desc(int rotary, int pairing, bool q, bool k, const float* c, const float* s) {
    atn_pe_desc d{};
    d.kind = ATN_PE_ROPE;
    d.pairing = pairing;
    d.rotary_dim = rotary;
    d.apply_q = q;
    d.apply_k = k;
    d.base = 10000.0f;
    d.table_a = c;
    d.table_b = s;
    return d;
}

atn_pe_desc sin_desc(bool q, bool k, const float* sin_t, const float* cos_t) {
    atn_pe_desc d{};
    d.kind = ATN_PE_SINUSOIDAL;
    d.apply_q = q;
    d.apply_k = k;
    d.table_a = sin_t;
    d.table_b = cos_t;
    return d;
}

}  // namespace

// ====================================================================== C ABI
extern "C" {

const char* atn_status_string(int status) {
    switch (status) {
        case ATN_OK: return "ok";
        case ATN_ERR_NULL_POINTER: return "null pointer";
        case ATN_ERR_BAD_DIMENSION: return "dimension < 1";
        case ATN_ERR_BAD_ROTARY: return "rotary_dim must be even and in [2, head_d]";
        case ATN_ERR_SIZE_OVERFLOW: return "size overflow";
        case ATN_ERR_ALIASING: return "output overlaps an input";
        case ATN_ERR_NO_DEVICE: return "no HIP device";
        case ATN_ERR_HIP: return "HIP runtime error";
        case ATN_ERR_WORKSPACE: return "workspace too small";
        case ATN_ERR_BAD_ARGUMENT: return "bad argument";
        case ATN_ERR_MISALIGNED: return "pointer not aligned to its element size";
        case ATN_ERR_DEVICE_TIMEOUT: return "device-side wait timed out (outputs are NaN)";
        case ATN_ERR_CAPTURE: return "library allocation needed while the stream is being captured";
        case ATN_ERR_SCRATCH_LIMIT:
            return "shape needs more scratch than the allocation-free entry point holds";
        case ATN_ERR_NOT_PREPARED:
            return "encoding tables not prepared (call atn_prepare_pe_ex first)";
        default: return "unknown status";
    }
}

int atn_last_hip_error(void) { return g_last_hip_error; }

int atn_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

int atn_set_tuning_ex(const atn_tuning* t) {
    std::unique_ptr<const atn_tuning> fresh(new atn_tuning(t ? *t : atn_tuning{}));
    atn::s16_set_tile(fresh->splitd_tile);
    std::lock_guard<std::mutex> tl(g_tune_mu);
    const atn_tuning* old = g_tune.exchange(fresh.release(), std::memory_order_acq_rel);
    g_tune_old.emplace_back(old);
    std::lock_guard<std::mutex> lk(g_mu);
    g_fused_plans.clear();
    return ATN_OK;
}

int atn_get_tuning_ex(atn_tuning* t) {
    if (!t) return ATN_ERR_NULL_POINTER;
    *t = tune();
    return ATN_OK;
}

int atn_fused_plan_ex(int dtype, int batch, int heads, int len_q, int len_k, int head_d,
                      const atn_pe_desc* pe, atn_fused_plan_info* info) {
    if (!info) return ATN_ERR_NULL_POINTER;
    if (dtype != ATN_DTYPE_F32 && dtype != ATN_DTYPE_BF16) return ATN_ERR_BAD_ARGUMENT;
    Shape s;
    int st = check_shape(batch, heads, len_q, len_k, head_d, &s);
    if (st != ATN_OK) return st;
    PePlan plan;
    st = check_pe(pe, head_d, &plan);
    if (st != ATN_OK) return st;
    *info = atn_fused_plan_info{};
    if (tune().no_fused) return 0;
    int n = 0;
    const bool dev = hipGetDeviceCount(&n) == hipSuccess && n > 0;
    const FusedPlan p = fused_plan(dtype, plan.pek, s, dev);
    if (!p.ok) return 0;
    info->rows = p.MB;
    info->dc = p.dc;
    info->nchunk = p.nchunk;
    info->gather1 = p.gather1;
    info->xcd = p.xcd;
    info->workgroups = p.workgroups;
    info->lds = p.lds;
    return 1;
}

long atn_rerun_count(int reset) {
    return reset ? g_reruns.exchange(0) : g_reruns.load();
}

size_t atn_retained_bytes_ex(void) {
    int dev;
    if (current_device(&dev) != ATN_OK) return 0;
    std::lock_guard<std::mutex> lk(g_mu);
    const DeviceState& ds = g_dev[dev];
    size_t b = ds.live_bytes;
    for (const auto& r : ds.retired) b += r.second;
    return b;
}

int atn_release_ex(void) {
    int dev;
    int st = current_device(&dev);
    if (st != ATN_OK) return st;
    std::lock_guard<std::mutex> lk(g_mu);
    DeviceState& ds = g_dev[dev];
    if (ds.retired.empty()) return ATN_OK;
    ATN_HIP(hipDeviceSynchronize());
    for (const auto& r : ds.retired) ATN_HIP(hipFree(r.first));
    ds.retired.clear();
    return ATN_OK;
}

int atn_attention_fwd_ex(int dtype, const void* Q, const void* K, const void* V, void* out,
                         int batch, int heads, int len_q, int len_k, int head_d,
                         const atn_pe_desc* pe, void* workspace, size_t workspace_bytes,
                         void* stream) {
    return attention_core(dtype, Q, K, V, out, batch, heads, len_q, len_k, head_d, pe, workspace,
                          workspace_bytes, (hipStream_t)stream);
}

int atn_attention_fwd_noalloc_ex(int dtype, const void* Q, const void* K, const void* V,
                                 void* out, int batch, int heads, int len_q, int len_k,
                                 int head_d, const atn_pe_desc* pe, void* stream) {
    return attention_core(dtype, Q, K, V, out, batch, heads, len_q, len_k, head_d, pe, nullptr, 0,
                          (hipStream_t)stream, true);
}

size_t atn_attention_workspace_bytes(int dtype, int batch, int heads, int len_q, int len_k,
                                     int head_d, const atn_pe_desc* pe) {
    if (dtype != ATN_DTYPE_F32 && dtype != ATN_DTYPE_BF16) return 0;
    Shape s;
    if (check_shape(batch, heads, len_q, len_k, head_d, &s) != ATN_OK) return 0;
    PePlan plan;
    if (check_pe(pe, head_d, &plan) != ATN_OK) return 0;
    // the largest workspace of every plan the call could take, or, when that
    // exceeds the library's cap, of the chunks the call then runs in
    const size_t full = path_need(dtype, s, plan, false, -1, -1);
    if (full <= library_cap()) return full;
    const Chunking ch = plan_chunks(dtype, s, plan, library_cap(), false, -1, -1);
    return ch.heads > 0 ? ch.need : full;
}

int atn_pe_apply_ex(int dtype, const void* in, void* out, long n_rows, int seq_len, int head_d,
                    const atn_pe_desc* pe, void* stream) {
    return pe_apply_core(dtype, in, out, n_rows, seq_len, head_d, pe, (hipStream_t)stream);
}

int atn_attention_path_ex(int dtype, int batch, int heads, int len_q, int len_k, int head_d,
                          const atn_pe_desc* pe) {
    if (dtype != ATN_DTYPE_F32 && dtype != ATN_DTYPE_BF16) return ATN_ERR_BAD_ARGUMENT;
    Shape s;
    int st = check_shape(batch, heads, len_q, len_k, head_d, &s);
    if (st != ATN_OK) return st;
    PePlan plan;
    st = check_pe(pe, head_d, &plan);
    if (st != ATN_OK) return st;
    int n = 0;
    const bool dev = hipGetDeviceCount(&n) == hipSuccess && n > 0;
    if (!tune().no_fused && fused_plan(dtype, plan.pek, s, dev).ok) return ATN_PATH_FUSED_SMALL;
    plan.no_flash = tune().no_flash != 0;
    if (flash_ok(dtype, s, plan)) return ATN_PATH_FLASH;
    if (gemm_plan(dtype, s, plan).ok) return ATN_PATH_GEMM;
    return ATN_PATH_SPLIT_D;
}

int atn_sync_status_ex(void* workspace, int batch, int heads, void* stream) {
    hipStream_t st = (hipStream_t)stream;
    int dev;
    int s = current_device(&dev);
    if (s != ATN_OK) return s;
    (void)batch;
    (void)heads;
    ATN_HIP(hipStreamSynchronize(st));
    return workspace_status(workspace, st);
}

int atn_prepare_pe_ex(const atn_pe_desc* pe, int head_d, int max_positions) {
    if (!pe) return ATN_ERR_NULL_POINTER;
    if (head_d < 1 || max_positions < 1) return ATN_ERR_BAD_DIMENSION;
    PePlan plan;
    int st = check_pe(pe, head_d, &plan);
    if (st != ATN_OK) return st;
    if (plan.pek == atn::kPeNone || plan.caller_tables) return ATN_OK;
    st = bind_tables(pe, plan, head_d, max_positions, nullptr);
    if (st != ATN_OK) return st;
    // and the fp16 tables of the GEMM path's in-GEMM K encoding
    int dev;
    st = current_device(&dev);
    if (st != ATN_OK) return st;
    std::lock_guard<std::mutex> lk(g_mu);
    Table16* t16 = nullptr;
    return get_table16(g_dev[dev], plan, head_d, max_positions, nullptr, false, &t16);
}

// ---- drop-ins ----
void attention_forward_optimized(const float* Q, const float* K, const float* V, float* out,
                                 int batch_sz, int num_heads, int len_q, int len_k, int head_d) {
    dropin_attention("attention_forward_optimized", ATN_DTYPE_F32, Q, K, V, out,
                     batch_sz, num_heads, len_q, len_k, head_d, nullptr);
}

void attention_forward(const float* Q, const float* K, const float* V, float* out, int batch_sz,
                       int num_heads, int len_q, int len_k, int head_d) {
    dropin_attention("attention_forward", ATN_DTYPE_F32, Q, K, V, out,
                     batch_sz, num_heads, len_q, len_k, head_d, nullptr);
}

void attention_forward_rope_fused(const float* Q, const float* K, const float* V, float* out,
                                  const float* cos_cache, const float* sin_cache, int batch_sz,
                                  int num_heads, int len_q, int len_k, int head_d) {
    if (!cos_cache || !sin_cache) die(ATN_ERR_NULL_POINTER, "attention_forward_rope_fused");
    const atn_pe_desc d = rope_desc(head_d, ATN_ROPE_INTERLEAVED, true, true, cos_cache, sin_cache);
    dropin_attention("attention_forward_rope_fused", ATN_DTYPE_F32, Q, K, V, out,
                     batch_sz, num_heads, len_q, len_k, head_d, &d);
}

void attention_forward_rope_fused_v7_hybrid(const float* Q, const float* K_rotated,
                                            const float* V, float* out, int batch_sz,
                                            int num_heads, int len_q, int len_k, int head_d,
                                            int rotary_dim) {
    const atn_pe_desc d = rope_desc(rotary_dim, ATN_ROPE_INTERLEAVED, true, false, nullptr, nullptr);
    if (rotary_dim == 0) die(ATN_ERR_BAD_ROTARY, "attention_forward_rope_fused_v7_hybrid");
    dropin_attention("attention_forward_rope_fused_v7_hybrid", ATN_DTYPE_F32, Q, K_rotated, V, out,
                     batch_sz, num_heads, len_q, len_k, head_d, &d);
}

void attention_forward_separate_rope(const float* Q, const float* K, const float* V,
                                     float* Q_rope, float* K_rope, float* out,
                                     const float* cos_cache, const float* sin_cache, int batch_sz,
                                     int num_heads, int len_q, int len_k, int head_d,
                                     int rotary_dim) {
    const char* w = "attention_forward_separate_rope";
    if (!cos_cache || !sin_cache || !Q_rope || !K_rope) die(ATN_ERR_NULL_POINTER, w);
    if (rotary_dim == 0) die(ATN_ERR_BAD_ROTARY, w);
    const atn_pe_desc d = rope_desc(rotary_dim, ATN_ROPE_INTERLEAVED, true, true, cos_cache, sin_cache);
    Shape s;
    int st = check_shape(batch_sz, num_heads, len_q, len_k, head_d, &s);
    if (st != ATN_OK) die(st, w);
    st = pe_apply_core(ATN_DTYPE_F32, Q, Q_rope, (long)(s.BH * len_q), len_q, head_d, &d, nullptr);
    if (st != ATN_OK) die(st, w);
    st = pe_apply_core(ATN_DTYPE_F32, K, K_rope, (long)(s.BH * len_k), len_k, head_d, &d, nullptr);
    if (st != ATN_OK) die(st, w);
    dropin_attention(w, ATN_DTYPE_F32, Q_rope, K_rope, V, out,
                     batch_sz, num_heads, len_q, len_k, head_d, nullptr);
}

void rope_forward(const float* input, float* output, const float* cos_cache,
                  const float* sin_cache, int total_tokens, int hdim, int rotary_dim,
                  int seq_len) {
    if (!cos_cache || !sin_cache) die(ATN_ERR_NULL_POINTER, "rope_forward");
    if (rotary_dim == 0) die(ATN_ERR_BAD_ROTARY, "rope_forward");
    const atn_pe_desc d = rope_desc(rotary_dim, ATN_ROPE_INTERLEAVED, true, true, cos_cache, sin_cache);
    sync_or_die(pe_apply_core(ATN_DTYPE_F32, input, output, total_tokens, seq_len, hdim, &d,
                              nullptr),
                "rope_forward");
}

void apply_sinusoidal_embeddings(const float* input, const float* sin_table,
                                 const float* cos_table, float* output, int total_tokens,
                                 int hdim, int seqlen) {
    if (!sin_table || !cos_table) die(ATN_ERR_NULL_POINTER, "apply_sinusoidal_embeddings");
    const atn_pe_desc d = sin_desc(true, true, sin_table, cos_table);
    sync_or_die(pe_apply_core(ATN_DTYPE_F32, input, output, total_tokens, seqlen, hdim, &d,
                              nullptr),
                "apply_sinusoidal_embeddings");
}

void attention_forward_sinusoidal_fused(const float* Q, const float* K, const float* V,
                                        float* out, int batch_sz, int num_heads, int len_q,
                                        int len_k, int head_d) {
    const atn_pe_desc d = sin_desc(true, true, nullptr, nullptr);
    dropin_attention("attention_forward_sinusoidal_fused", ATN_DTYPE_F32, Q, K, V, out,
                     batch_sz, num_heads, len_q, len_k, head_d, &d);
}

void attention_forward_sinusoidal_hybrid(const float* Q, const float* K, const float* V,
                                         const float* sin_table, const float* cos_table,
                                         float* K_emb, float* out, int batch_sz, int num_heads,
                                         int len_q, int len_k, int head_d) {
    const char* w = "attention_forward_sinusoidal_hybrid";
    if (!sin_table || !cos_table || !K_emb) die(ATN_ERR_NULL_POINTER, w);
    Shape s;
    int st = check_shape(batch_sz, num_heads, len_q, len_k, head_d, &s);
    if (st != ATN_OK) die(st, w);
    const atn_pe_desc dk = sin_desc(true, true, sin_table, cos_table);
    st = pe_apply_core(ATN_DTYPE_F32, K, K_emb, (long)(s.BH * len_k), len_k, head_d, &dk, nullptr);
    if (st != ATN_OK) die(st, w);
    const atn_pe_desc dq = sin_desc(true, false, sin_table, cos_table);
    dropin_attention(w, ATN_DTYPE_F32, Q, K_emb, V, out,
                     batch_sz, num_heads, len_q, len_k, head_d, &dq);
}

void attention_forward_sinusoidal_separate(const float* Q, const float* K, const float* V,
                                           const float* sin_table, const float* cos_table,
                                           float* Q_emb, float* K_emb, float* out, int batch_sz,
                                           int num_heads, int len_q, int len_k, int head_d) {
    const char* w = "attention_forward_sinusoidal_separate";
    if (!sin_table || !cos_table || !Q_emb || !K_emb) die(ATN_ERR_NULL_POINTER, w);
    Shape s;
    int st = check_shape(batch_sz, num_heads, len_q, len_k, head_d, &s);
    if (st != ATN_OK) die(st, w);
    const atn_pe_desc d = sin_desc(true, true, sin_table, cos_table);
    st = pe_apply_core(ATN_DTYPE_F32, Q, Q_emb, (long)(s.BH * len_q), len_q, head_d, &d, nullptr);
    if (st != ATN_OK) die(st, w);
    st = pe_apply_core(ATN_DTYPE_F32, K, K_emb, (long)(s.BH * len_k), len_k, head_d, &d, nullptr);
    if (st != ATN_OK) die(st, w);
    dropin_attention(w, ATN_DTYPE_F32, Q_emb, K_emb, V, out,
                     batch_sz, num_heads, len_q, len_k, head_d, nullptr);
}

void attention_forward_bf16(const atn_bf16* Q, const atn_bf16* K, const atn_bf16* V,
                            atn_bf16* out, int bs, int nh, int len_q, int len_k, int head_d) {
    dropin_attention("attention_forward_bf16", ATN_DTYPE_BF16, Q, K, V, out,
                     bs, nh, len_q, len_k, head_d, nullptr);
}

void attention_forward_rope_bf16(const atn_bf16* Q, const atn_bf16* K_rotated,
                                 const atn_bf16* V, atn_bf16* out, int bs, int nh, int len_q,
                                 int len_k, int head_d, int rotary_dim) {
    if (rotary_dim == 0) die(ATN_ERR_BAD_ROTARY, "attention_forward_rope_bf16");
    const atn_pe_desc d = rope_desc(rotary_dim, ATN_ROPE_INTERLEAVED, true, false, nullptr, nullptr);
    dropin_attention("attention_forward_rope_bf16", ATN_DTYPE_BF16, Q, K_rotated, V, out,
                     bs, nh, len_q, len_k, head_d, &d);
}

void attention_forward_rope_fused_bf16(const atn_bf16* Q, const atn_bf16* K, const atn_bf16* V,
                                       atn_bf16* out, int bs, int nh, int len_q, int len_k,
                                       int head_d) {
    const atn_pe_desc d = rope_desc(head_d, ATN_ROPE_INTERLEAVED, true, true, nullptr, nullptr);
    dropin_attention("attention_forward_rope_fused_bf16", ATN_DTYPE_BF16, Q, K, V, out,
                     bs, nh, len_q, len_k, head_d, &d);
}

void attention_forward_sinusoidal_bf16(const atn_bf16* Q, const atn_bf16* K, const atn_bf16* V,
                                       atn_bf16* out, int bs, int nh, int len_q, int len_k,
                                       int head_d) {
    const atn_pe_desc d = sin_desc(true, true, nullptr, nullptr);
    dropin_attention("attention_forward_sinusoidal_bf16", ATN_DTYPE_BF16, Q, K, V, out,
                     bs, nh, len_q, len_k, head_d, &d);
}

void precompute_rope_cache(float* cos_cache, float* sin_cache, int max_seq_len, int rotary_dim,
                           float base) {
    // final/rope.cu:20-40
    for (int pos = 0; pos < max_seq_len; pos++) {
        for (int i = 0; i < rotary_dim / 2; i++) {
            const float freq = 1.0f / powf(base, (2.0f * i) / rotary_dim);
            const float theta = pos * freq;
            const float c = cosf(theta), s = sinf(theta);
            cos_cache[(size_t)pos * rotary_dim + 2 * i] = c;
            cos_cache[(size_t)pos * rotary_dim + 2 * i + 1] = c;
            sin_cache[(size_t)pos * rotary_dim + 2 * i] = s;
            sin_cache[(size_t)pos * rotary_dim + 2 * i + 1] = s;
        }
    }
}

void precompute_sinusoidal_table(float* sin_table, float* cos_table, int seqlen, int hdim) {
    // final/sinusoidal.cu:838-855
    for (int pos = 0; pos < seqlen; pos++) {
        for (int d = 0; d < hdim; d++) {
            const float freq = 1.0f / powf(10000.0f, (2.0f * (d / 2)) / (float)hdim);
            const float angle = pos * freq;
            sin_table[(size_t)pos * hdim + d] = sinf(angle);
            cos_table[(size_t)pos * hdim + d] = cosf(angle);
        }
    }
}

}  // extern "C"
