// Row softmax for gfx950, plain and in the scaled, length-masked form of attention scores.
//
// Semantics: cpu_ref::softmax (reference src/backend/cpu_ref/ops.cpp:644-661): peak = max, sum = sum exp(x - peak),
// y = exp(x - peak) / sum, all in f64, rounded once to f32. The masked form is what cpu-ref evaluates for
// Softmax(Add(Scale(s, scale), mask)) with a 0/-inf key mask: s * scale in f32 (ops.cpp:209-211), -inf on masked keys,
// which come out exactly 0. (Device analog: sycl_be::softmax, src/backend/sycl/sycl_kernels.cpp:1071-1090, and the
// masked attention_softmax, :2047-2104.)
//
// Layout: as the row norms, LPR lanes share a row (16..1024) and hold it in registers (up to NV 128-bit vectors per
// lane), so the row is read from HBM once and written once, and exp is evaluated once per element. Reductions: the max
// in f32 (exact) by DPP within a wave and one LDS stage across waves; x - peak carries its rounding error (TwoSum) into
// exp; the sum is accumulated in f64; y = e * (1 / sum) in f64, rounded once. Masked keys are neither loaded nor
// exponentiated.
//
// Few wide rows (the decode step's [heads, 1, keys] scores) would leave most of the chip idle with one workgroup per
// row, so with caller scratch a row is split over `chunks` workgroups in ONE launch: each reduces its chunk to
// (max m_j, f64 sum s_j of exp(x - m_j)), publishes it through the scratch with device-scope atomics, waits for the
// row's other chunks (a bounded wait, with a local fallback), combines the row's partials and writes its chunk's
// outputs from the values it still holds in registers -- the scores are read from HBM once and written once.
#include <cmath>

#include "common.h"

namespace xs_hip {
namespace {

struct SoftmaxArgs {
    const float* x;
    float* y;
    int64_t rows, width, row_stride;
    float scale;
    const int64_t* valid_len;  // per row, or null
    int64_t valid_all;
};

// exp(s - peak) with the rounding error of the f32 subtraction folded back in: d + err == s - peak exactly (TwoSum,
// Knuth), and exp(d + err) = exp(d) (1 + err) to first order.
__device__ __forceinline__ float exp_diff(float s, float peak) {
    const float d = s - peak;
    const float bb = d - s;
    const float err = (s - (d - bb)) + (-peak - bb);
    const float e = expf(d);
    return (err != 0.0f && err == err) ? fmaf(e, err, e) : e;
}

template <int LPR, int NV>
__global__ __launch_bounds__(LPR > kBlock ? LPR : kBlock) void softmax_vec(SoftmaxArgs p) {
    constexpr int BLOCK = LPR > kBlock ? LPR : kBlock;
    constexpr int ROWS_PER_BLOCK = BLOCK / LPR;
    constexpr int WAVES_PER_ROW = LPR > 64 ? LPR / 64 : 1;
    constexpr int W = LPR < 64 ? LPR : 64;
    __shared__ float part_max[BLOCK / 64];
    __shared__ double part_sum[BLOCK / 64];

    const int l = threadIdx.x % LPR;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * ROWS_PER_BLOCK + threadIdx.x / LPR;
    const bool live = row < p.rows;
    const int64_t nvec = p.width / 4;
    int64_t valid = p.valid_len != nullptr && live ? p.valid_len[row] : p.valid_all;
    valid = valid < 0 ? 0 : (valid > p.width ? p.width : valid);
    const float* xr = p.x + row * p.row_stride;

    float s[NV][4];
    u32x4 raw[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int64_t v = l + static_cast<int64_t>(k) * LPR;
        if (live && v < nvec && v * 4 < valid) raw[k] = ld128_nt(xr + v * 4);
    }
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int64_t v = l + static_cast<int64_t>(k) * LPR;
        if (live && v < nvec && v * 4 < valid) {
            unpack<F32>(raw[k], s[k]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                s[k][i] = v * 4 + i < valid ? s[k][i] * p.scale : -INFINITY;
                m = fmaxf(m, s[k][i]);
            }
        }
    }
    m = group_reduce<W, OpMax>(m);
    if constexpr (WAVES_PER_ROW > 1) {
        const int wave = threadIdx.x >> 6;
        if ((threadIdx.x & 63) == 0) part_max[wave] = m;
        __syncthreads();
        const int first = (wave / WAVES_PER_ROW) * WAVES_PER_ROW;
        m = part_max[first];
#pragma unroll
        for (int i = 1; i < WAVES_PER_ROW; ++i) m = fmaxf(m, part_max[first + i]);
    }
    // A row whose keys are all masked or -inf has peak -inf and exp(-inf - -inf) = NaN, as in cpu-ref; with nothing
    // loaded the sum stays 0 and 0 * (1 / 0) below is NaN too. A NaN sum makes every output NaN, masked keys included
    // (cpu-ref divides their exp(-inf) = 0 by it).
    double sum = 0.0;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int64_t v = l + static_cast<int64_t>(k) * LPR;
        if (live && v < nvec && v * 4 < valid) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                s[k][i] = v * 4 + i < valid ? exp_diff(s[k][i], m) : 0.0f;
                sum += static_cast<double>(s[k][i]);
            }
        }
    }
    sum = group_sum_f64<W>(sum);
    if constexpr (WAVES_PER_ROW > 1) {
        const int wave = threadIdx.x >> 6;
        if ((threadIdx.x & 63) == 0) part_sum[wave] = sum;
        __syncthreads();
        const int first = (wave / WAVES_PER_ROW) * WAVES_PER_ROW;
        sum = 0.0;
#pragma unroll
        for (int i = 0; i < WAVES_PER_ROW; ++i) sum += part_sum[first + i];
    }
    if (!live) return;
    const double rinv = 1.0 / sum;
    float* yr = p.y + row * p.row_stride;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int64_t v = l + static_cast<int64_t>(k) * LPR;
        if (v < nvec) {
            float o[4];
            const float masked = static_cast<float>(0.0 * rinv);
            if (v * 4 < valid) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    o[i] = v * 4 + i < valid ? static_cast<float>(static_cast<double>(s[k][i]) * rinv) : masked;
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) o[i] = masked;
            }
            st128_nt(yr + v * 4, pack<F32>(o));
        }
    }
}

// Any width or alignment: one block per row, three passes over the row (the later ones from cache).
__global__ __launch_bounds__(kBlock) void softmax_any(SoftmaxArgs p) {
    __shared__ float part_max[kBlock / 64];
    __shared__ double part_sum[kBlock / 64];
    const int64_t row = blockIdx.x;
    int64_t valid = p.valid_len != nullptr ? p.valid_len[row] : p.valid_all;
    valid = valid < 0 ? 0 : (valid > p.width ? p.width : valid);
    const float* xr = p.x + row * p.row_stride;
    float* yr = p.y + row * p.row_stride;
    float m = -INFINITY;
    for (int64_t i = threadIdx.x; i < valid; i += kBlock) m = fmaxf(m, xr[i] * p.scale);
    m = group_reduce<64, OpMax>(m);
    if ((threadIdx.x & 63) == 0) part_max[threadIdx.x >> 6] = m;
    __syncthreads();
    m = part_max[0];
    for (int i = 1; i < kBlock / 64; ++i) m = fmaxf(m, part_max[i]);
    double sum = 0.0;
    for (int64_t i = threadIdx.x; i < valid; i += kBlock) sum += static_cast<double>(exp_diff(xr[i] * p.scale, m));
    sum = group_sum_f64<64>(sum);
    if ((threadIdx.x & 63) == 0) part_sum[threadIdx.x >> 6] = sum;
    __syncthreads();
    sum = 0.0;
    for (int i = 0; i < kBlock / 64; ++i) sum += part_sum[i];
    const double rinv = 1.0 / sum;
    const float masked = static_cast<float>(0.0 * rinv);
    // Read every input of the row before the first write: y may alias x.
    __syncthreads();
    for (int64_t i = threadIdx.x; i < p.width; i += kBlock) {
        yr[i] = i < valid ? static_cast<float>(static_cast<double>(exp_diff(xr[i] * p.scale, m)) * rinv)
                          : masked;
    }
}

constexpr int kMaxChunks = 64;       // one wave combines a row's partials, a chunk a lane
__device__ __forceinline__ int64_t row_valid(const SoftmaxArgs& p, int64_t row) {
    const int64_t v = p.valid_len != nullptr ? p.valid_len[row] : p.valid_all;
    return v < 0 ? 0 : (v > p.width ? p.width : v);
}

// The scaled keys of one chunk (VPT 128-bit vectors a lane, lane t holding vectors t + k * BLOCK of the chunk), -inf
// for masked ones and past the row. Plain loads: at a few KiB a workgroup the load latency is the cost, and the
// non-temporal form measured slower there.
template <int BLOCK, int VPT>
__device__ __forceinline__ void load_chunk(const SoftmaxArgs& p, int64_t row, int chunk, int64_t valid,
                                           float (&s)[VPT][4]) {
    const float* xr = p.x + row * p.row_stride;
    const int64_t v0 = static_cast<int64_t>(chunk) * (BLOCK * VPT);
    const int64_t nvec = p.width / 4;
    u32x4 raw[VPT];
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int64_t v = v0 + threadIdx.x + k * BLOCK;
        if (v < nvec && v * 4 < valid) raw[k] = ld128(xr + v * 4);
    }
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int64_t v = v0 + threadIdx.x + k * BLOCK;
        if (v < nvec && v * 4 < valid) {
            unpack<F32>(raw[k], s[k]);
#pragma unroll
            for (int i = 0; i < 4; ++i) s[k][i] = v * 4 + i < valid ? s[k][i] * p.scale : -INFINITY;
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) s[k][i] = -INFINITY;
        }
    }
}

// exp(a - b) for a <= b as f64: in f32 with the subtraction's rounding error folded in while the result is a normal
// f32 (a - b >= -80), else in f64.
__device__ __forceinline__ double exp_gap(float a, float b) {
    return a - b >= -80.0f ? static_cast<double>(exp_diff(a, b))
                           : exp(static_cast<double>(a) - static_cast<double>(b));
}

// Partials of one chunk held in registers. Each wave takes its own maximum m_w and replaces its values by
// exp(x - m_w), summed in f32 (s_w); one LDS stage hands the waves' (m_w, s_w) to wave 0, whose lane w holds wave w's
// pair: m_j = max m_w and s_j = sum s_w exp(m_w - m_j) in f64, returned wave-uniform in wave 0 (the other waves'
// m_j, s_j are unspecified). A wave whose keys are all masked or -inf has m_w = -inf, exponentials 0 and adds
// nothing (its exponentials relative to its own -inf maximum would be NaN). Every reduction runs in a fixed order, so
// the same chunk gives the same bits in any workgroup. The LDS arrays are read after the barrier: a caller that
// reuses them puts a barrier before the next call.
template <int BLOCK, int VPT>
__device__ __forceinline__ void chunk_stats(float (&s)[VPT][4], float* lds_m, float* lds_s, float& m_w, float& m_j,
                                            double& s_j) {
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < VPT; ++k)
#pragma unroll
        for (int i = 0; i < 4; ++i) m = fmaxf(m, s[k][i]);
    m_w = wave_reduce<OpMax>(m, -INFINITY);
    float lane_sum = 0.0f;
#pragma unroll
    for (int k = 0; k < VPT; ++k)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            s[k][i] = m_w != -INFINITY ? exp_diff(s[k][i], m_w) : 0.0f;
            lane_sum += s[k][i];
        }
    const float s_w = wave_reduce<OpSum>(lane_sum, 0.0f);
    constexpr int kWaves = BLOCK / 64;
    if ((threadIdx.x & 63) == 0) {
        lds_m[threadIdx.x >> 6] = m_w;
        lds_s[threadIdx.x >> 6] = s_w;
    }
    lds_barrier();
    if (threadIdx.x < 64) {
        const int l = threadIdx.x;
        const float mw = l < kWaves ? lds_m[l] : -INFINITY;
        const float sw = l < kWaves ? lds_s[l] : 0.0f;
        const float mx = group_reduce<kWaves, OpMax>(mw);
        const double sx = group_sum_f64<kWaves>(mw != -INFINITY ? static_cast<double>(sw) * exp_gap(mw, mx) : 0.0);
        m_j = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(mx)));
        const uint64_t u = __double_as_longlong(sx);
        s_j = __longlong_as_double(static_cast<int64_t>(
            (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(u >> 32))))
             << 32) |
            static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(u)))));
    }
}

// Wave 0, lane j holding chunk j's partial (m_l, s_l): the row's M = max m_j and 1 / S, S = sum s_j exp(m_j - M) in
// f64, into LDS. M = -inf (every key masked or -inf) makes S NaN, as cpu-ref's exp(-inf - (-inf)) makes the row NaN.
__device__ __forceinline__ void combine_row(float m_l, double s_l, int chunks, float* s_M, double* s_rS) {
    const int lane = threadIdx.x;
    const float M = wave_reduce<OpMax>(lane < chunks ? m_l : -INFINITY, -INFINITY);
    const double t = lane >= chunks     ? 0.0
                     : m_l != -INFINITY ? s_l * exp_gap(m_l, M)
                                        : (M == -INFINITY ? NAN : 0.0);
    const double S = wave_sum_f64(t);
    if (lane == 0) {
        *s_M = M;
        *s_rS = 1.0 / S;
    }
}

// Scratch of the split launch, all 64-bit words, zero-filled before its first use. Row r owns a fixed block of
// kRowWords words whatever the call's shape (so calls of any shapes can follow each other on one scratch):
//   word 0: the row's ticket counter, (generation << 32) | tickets taken this call;
//   words 8 + 128 b ..: bank b of partial pairs, chunk j at 2 j: (m_j bits | 1 << 32, s_j bits ^ 1 << 63), never 0
//   once written, so a zero word means "not yet published" and a reader needs no ordering between the two words.
// A call uses bank (generation & 1); every workgroup of the row takes a ticket first, and the one that takes the
// row's last ticket rolls the counter to the next generation and clears the other bank -- the previous call's, whose
// readers are all done, since that call's kernel has ended -- so the next call finds its bank zero, and nothing is
// left to do at the end of the kernel. Every access is a relaxed device-scope atomic, which this part keeps coherent
// across the XCDs' L2s without cache write-back or invalidation.
constexpr int kMaxSplitRows = 256;  // a split launch has fewer than 256 rows
constexpr int64_t kBankWords = 2 * kMaxChunks;
constexpr int64_t kRowWords = 8 + 2 * kBankWords;

__device__ __forceinline__ uint64_t enc_max(float m) { return (uint64_t{1} << 32) | __float_as_uint(m); }
__device__ __forceinline__ uint64_t enc_sum(double s) {
    return static_cast<uint64_t>(__double_as_longlong(s)) ^ (uint64_t{1} << 63);
}
__device__ __forceinline__ float dec_max(uint64_t w) { return __uint_as_float(static_cast<uint32_t>(w)); }
__device__ __forceinline__ double dec_sum(uint64_t w) {
    return __longlong_as_double(static_cast<long long>(w ^ (uint64_t{1} << 63)));
}
__device__ __forceinline__ uint64_t ld_sync(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_sync(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One launch, grid (chunks, rows) of BLOCK threads, chunk = BLOCK * VPT * 4 keys. Each workgroup reduces its chunk
// to (m_j, s_j), keeping the chunk's exp(x - m_j) in registers, publishes the pair, waits (at most `spin` polls) for
// the row's other chunks, combines the row's partials -- M = max m_j, S = sum s_j exp(m_j - M) in f64, lane j holding
// chunk j so every workgroup adds them in one order -- and writes its chunk's exp(x - m_j) * (exp(m_j - M) / S): the
// scores are read once and exponentiated once. A workgroup whose wait runs out (its row's chunks not all resident:
// another kernel holding the CUs, or the spin limit a test sets) computes every chunk's partial of its row itself with
// the same reductions, so its result has the same bits, and still departs.
template <int BLOCK, int VPT>
__global__ __launch_bounds__(BLOCK) void softmax_split(SoftmaxArgs p, int chunks, uint64_t* __restrict__ sync,
                                                       int spin) {
    __shared__ float lds_m[BLOCK / 64];
    __shared__ float lds_s[BLOCK / 64];
    __shared__ float s_M;
    __shared__ double s_rS;
    __shared__ int s_ready;
    const int64_t row = blockIdx.y;
    const int chunk = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const bool wave0 = threadIdx.x < 64;
    uint64_t* rb = sync + row * kRowWords;
    const int64_t valid = row_valid(p, row);
    // The ticket comes back while the chunk loads.
    uint64_t ticket = 0;
    if (threadIdx.x == 0)
        ticket = __hip_atomic_fetch_add(rb, uint64_t{1}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    float s[VPT][4];
    load_chunk<BLOCK, VPT>(p, row, chunk, valid, s);
    float mw, mj;
    double sj;
    chunk_stats<BLOCK, VPT>(s, lds_m, lds_s, mw, mj, sj);
    uint64_t* slots = rb;
    if (wave0) {
        ticket = __shfl(ticket, 0, 64);
        const uint64_t bank = (ticket >> 32) & 1;
        slots = rb + 8 + bank * kBankWords;
        if (lane == 0) {
            __hip_atomic_store(slots + 2 * chunk, enc_max(mj), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(slots + 2 * chunk + 1, enc_sum(sj), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (static_cast<uint32_t>(ticket) == static_cast<uint32_t>(chunks - 1)) {
            // The row's last ticket: the next generation, and the other bank cleared for it.
            if (lane == 0)
                __hip_atomic_fetch_add(rb, (uint64_t{1} << 32) - static_cast<uint64_t>(chunks), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            uint64_t* other = rb + 8 + (bank ^ 1) * kBankWords;
            st_sync(other + lane, 0);
            st_sync(other + 64 + lane, 0);
        }
    }
    // Wave 0 polls the row's partials, lane j reading chunk j's pair, and combines them once all are there.
    if (wave0) {
        bool ready = false;
        for (int it = 0; it < spin; ++it) {
            uint64_t w0 = 1, w1 = 1;
            if (lane < chunks) {
                w0 = ld_sync(slots + 2 * lane);
                w1 = ld_sync(slots + 2 * lane + 1);
            }
            if (__all(w0 != 0 && w1 != 0)) {
                combine_row(dec_max(w0), dec_sum(w1), chunks, &s_M, &s_rS);
                ready = true;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (lane == 0) s_ready = ready ? 1 : 0;
    }
    lds_barrier();
    if (!s_ready) {
        // Fallback: every chunk of the row from x, a chunk at a time, wave 0's lane j keeping chunk j's partial.
        float m_l = -INFINITY;
        double s_l = 0.0;
        for (int j = 0; j < chunks; ++j) {
            lds_barrier();  // the previous chunk's LDS reads are done
            float t[VPT][4];
            load_chunk<BLOCK, VPT>(p, row, j, valid, t);
            float tw, m;
            double sum;
            chunk_stats<BLOCK, VPT>(t, lds_m, lds_s, tw, m, sum);
            if (lane == j) {
                m_l = m;
                s_l = sum;
            }
        }
        if (wave0) combine_row(m_l, s_l, chunks, &s_M, &s_rS);
        lds_barrier();
    }
    // This wave's factor exp(m_w - M) / S; a NaN sum (NaN keys, or every key masked) makes every output NaN, masked
    // ones too.
    const double factor = (mw != -INFINITY ? exp_gap(mw, s_M) : 0.0) * s_rS;
    float* yr = p.y + row * p.row_stride;
    const int64_t v0 = static_cast<int64_t>(chunk) * (BLOCK * VPT);
    const int64_t nvec = p.width / 4;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int64_t v = v0 + threadIdx.x + k * BLOCK;
        if (v < nvec) {
            float o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = static_cast<float>(static_cast<double>(s[k][i]) * factor);
            st128_nt(yr + v * 4, pack<F32>(o));
        }
    }
}

// The split launch's shape: 1024-thread workgroups (16 waves: the per-element work of a chunk spread thin, one LDS
// stage for the chunk's partial), VPT vectors a lane, and at most max_blocks workgroups -- half of what the chip holds
// at once at the kernel's register count (one 1024-thread workgroup a CU at up to 128 registers, two at up to 64),
// so every chunk of a row is resident while its row waits. block 0 = no split. Measured at config 2a's 32 rows of
// 32768 (the rest of the shapes within 8%): 8 chunks a row of 4096 keys in 1024 threads 5.8-6.0 us a call; 16 chunks
// of 2048 in 512 threads 6.4 us; 8 of 4096 in 512 threads (two vectors a lane) 6.5 us; 32 of 1024 in 256 threads
// 12.7 us (the wait for the row's partials grows with the pollers and chunks).
struct SplitShape {
    int block = 0, vpt = 0;
    int64_t max_blocks = 0;
    int64_t chunk() const { return static_cast<int64_t>(block) * vpt * 4; }
};
constexpr SplitShape kSplitShapes[] = {{1024, 1, 256}, {1024, 2, 128}, {1024, 4, 128}};

// A row is split only when its one-workgroup form would leave the chip mostly idle (fewer than kMaxSplitRows rows),
// into the smallest chunks that keep the launch within its shape's max_blocks and a row within kMaxChunks chunks.
SplitShape split_shape(int64_t rows, int64_t width) {
    if (width % 4 != 0 || rows >= kMaxSplitRows) return {};
    for (const SplitShape& sh : kSplitShapes) {
        const int64_t chunks = (width + sh.chunk() - 1) / sh.chunk();
        if (chunks < 2) return {};
        if (chunks <= kMaxChunks && rows * chunks <= sh.max_blocks) return sh;
    }
    return {};
}

int64_t split_chunks(int64_t width, const SplitShape& sh) { return (width + sh.chunk() - 1) / sh.chunk(); }

size_t split_scratch_bytes(int64_t rows) { return static_cast<size_t>(rows * kRowWords) * 8; }

// Polls a split workgroup makes before computing its row alone (a test sets it small to take that path).
int g_spin_limit = 1 << 14;

template <int LPR>
int go_vec(hipStream_t s, const SoftmaxArgs& p, int nv) {
    constexpr int BLOCK = LPR > kBlock ? LPR : kBlock;
    const unsigned grid = static_cast<unsigned>((p.rows + (BLOCK / LPR) - 1) / (BLOCK / LPR));
    switch (nv) {
        case 1: softmax_vec<LPR, 1><<<grid, BLOCK, 0, s>>>(p); break;
        case 2: softmax_vec<LPR, 2><<<grid, BLOCK, 0, s>>>(p); break;
        case 3: softmax_vec<LPR, 3><<<grid, BLOCK, 0, s>>>(p); break;
        case 4: softmax_vec<LPR, 4><<<grid, BLOCK, 0, s>>>(p); break;
        case 5: softmax_vec<LPR, 5><<<grid, BLOCK, 0, s>>>(p); break;
        case 6: softmax_vec<LPR, 6><<<grid, BLOCK, 0, s>>>(p); break;
        case 7: softmax_vec<LPR, 7><<<grid, BLOCK, 0, s>>>(p); break;
        default: softmax_vec<LPR, 8><<<grid, BLOCK, 0, s>>>(p); break;
    }
    return check_launch("xs_hip_softmax");
}

constexpr int kMaxNv = 8;

int launch_softmax(hipStream_t s, const SoftmaxArgs& p, void* scratch) {
    if (p.rows == 0) return XS_HIP_OK;
    const SplitShape sh = split_shape(p.rows, p.width);
    if (scratch != nullptr && sh.block > 0 && aligned16(p.x) && aligned16(p.y) && p.row_stride % 4 == 0) {
        if (reinterpret_cast<uintptr_t>(scratch) % 16 != 0)
            return fail(XS_HIP_EINVAL, "xs_hip_softmax_masked: scratch must be 16-byte aligned");
        auto* sync = static_cast<uint64_t*>(scratch);
        const int chunks = static_cast<int>(split_chunks(p.width, sh));
        const dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(p.rows));
        const int sp = g_spin_limit;
        switch (sh.vpt) {
            case 1: softmax_split<1024, 1><<<grid, 1024, 0, s>>>(p, chunks, sync, sp); break;
            case 2: softmax_split<1024, 2><<<grid, 1024, 0, s>>>(p, chunks, sync, sp); break;
            default: softmax_split<1024, 4><<<grid, 1024, 0, s>>>(p, chunks, sync, sp); break;
        }
        return check_launch("xs_hip_softmax_masked");
    }
    // The in-register kernel needs whole 128-bit vectors; the three-pass kernel handles y aliasing x by reading the
    // row before writing it, the in-register one trivially (each lane reads its values before writing them).
    const bool vec = p.width % 4 == 0 && p.row_stride % 4 == 0 && aligned16(p.x) && aligned16(p.y);
    const int64_t nvec = p.width / 4;
    if (vec) {
        for (int lpr = 16; lpr <= 1024; lpr *= 2) {
            const int64_t nv = (nvec + lpr - 1) / lpr;
            if (nv > kMaxNv) continue;
            const int n = static_cast<int>(nv);
            switch (lpr) {
                case 16: return go_vec<16>(s, p, n);
                case 32: return go_vec<32>(s, p, n);
                case 64: return go_vec<64>(s, p, n);
                case 128: return go_vec<128>(s, p, n);
                case 256: return go_vec<256>(s, p, n);
                case 512: return go_vec<512>(s, p, n);
                default: return go_vec<1024>(s, p, n);
            }
        }
    }
    softmax_any<<<static_cast<unsigned>(p.rows), kBlock, 0, s>>>(p);
    return check_launch("xs_hip_softmax");
}

}  // namespace
}  // namespace xs_hip

using namespace xs_hip;

extern "C" {

int xs_hip_softmax(void* stream, const float* x, float* y, int64_t rows, int64_t width) {
    if (rows < 0 || width <= 0 || rows > 0x7fffffffLL)
        return fail(XS_HIP_EINVAL, "xs_hip_softmax: " + std::to_string(rows) + " rows of width " + std::to_string(width));
    if (rows == 0) return XS_HIP_OK;
    if (x == nullptr || y == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_softmax: null buffer");
    const SoftmaxArgs p{x, y, rows, width, width, 1.0f, nullptr, width};
    return launch_softmax(as_stream(stream), p, nullptr);
}

size_t xs_hip_softmax_scratch(int64_t rows, int64_t width) {
    if (rows <= 0 || width <= 0) return 0;
    const SplitShape sh = split_shape(rows, width);
    return sh.block > 0 ? split_scratch_bytes(rows) : 0;
}

int xs_hip_softmax_masked(void* stream, const float* x, float* y, int64_t rows, int64_t width, int64_t row_stride,
                          float scale, const int64_t* valid_len, int64_t valid_len_all, void* scratch) {
    if (rows < 0 || width <= 0 || rows > 0x7fffffffLL || row_stride < width)
        return fail(XS_HIP_EINVAL, "xs_hip_softmax_masked: " + std::to_string(rows) + " rows of width " +
                                       std::to_string(width) + " with row stride " + std::to_string(row_stride));
    if (rows == 0) return XS_HIP_OK;
    if (x == nullptr || y == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_softmax_masked: null buffer");
    const SoftmaxArgs p{x, y, rows, width, row_stride, scale, valid_len, valid_len_all};
    return launch_softmax(as_stream(stream), p, scratch);
}

void xs_hip_set_spin_limit(int polls) { g_spin_limit = polls < 0 ? 0 : polls; }

}  // extern "C"
