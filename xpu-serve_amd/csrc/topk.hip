// Top-k along the last axis for gfx950, with the vocabulary-wide argmax (k = 1) as the fast path.
//
// Semantics: cpu_ref::topk (reference src/backend/cpu_ref/ops.cpp:663-684): values and i32 indices of the k largest,
// largest first; equal values keep the lower index first (its partial_sort comparator
// in[a] > in[b] || (in[a] == in[b] && a < b); spec src/graph/graph.h:70-71). k = 1 is blocks::argmax_rows
// (src/models/common/blocks.cpp:36-38). Launchers replaced: sycl_be::topk_scratch / topk
// (src/backend/sycl/sycl_kernels.h:61-63; sycl_kernels.cpp:1092-1254).
//
// Order used everywhere here: (v, i) precedes (w, j) when v > w, or v == w and i < j. It is a strict total order on
// non-NaN values (+0 and -0 compare equal, so the lower index wins, and the winner's own bits are reported). NaN is
// never selected; a row with fewer than k non-NaN values reports index 0 and x[0] for the missing places (cpu-ref's
// comparator is not a strict weak order with NaN, so its result there is unspecified).
//
// k = 1: a row is cut into chunks of kChunk values; a block reduces one chunk (one 128-bit load per lane, DPP within
// waves, one LDS stage across waves). A row of one chunk is done there; otherwise each chunk's (value, index) goes to
// scratch and a second launch, one block per row, reduces the row's partials -- no atomics and no waiting between
// workgroups.
// k > 1, rows up to 4096 wide (MoE routers, centroids): a wave per row holds the row in registers and picks the k
// winners one after another, each the wave's largest remaining element. Wider rows (a shortlist of a vocabulary, a
// drafter's candidates): a histogram of the row's top 11 key bits finds the bin of the k-th largest, everything from
// that bin up is compacted (a few hundred elements, typically), and one workgroup ranks those; a row whose bin is too
// crowded, or that holds fewer than k non-NaN values, is selected by k passes over it, with the same result.
#include <cfloat>
#include <climits>

#include "common.h"

namespace xs_hip {
namespace {

constexpr int kChunk = 1024;  // values per block for k = 1: one 128-bit vector per lane
constexpr int64_t kMaxRows = 65535;  // grid.y

// A (value, index) partial as one 64-bit word: the value's bits low, the index high, so it moves with one atomic.
__device__ __forceinline__ uint64_t pack_best(float v, int32_t i) {
    return static_cast<uint64_t>(__float_as_uint(v)) | (static_cast<uint64_t>(static_cast<uint32_t>(i)) << 32);
}

// true when (v, i) precedes (bv, bi).
__device__ __forceinline__ bool better(float v, int32_t i, float bv, int32_t bi) {
    return v > bv || (v == bv && i < bi);
}

template <int Ctrl>
__device__ __forceinline__ void dpp_best(float& v, int32_t& i) {
    const float ov = dpp_f<Ctrl>(v);
    const int32_t oi = dpp_i<Ctrl>(i);
    if (better(ov, oi, v, i)) {
        v = ov;
        i = oi;
    }
}

// Best over the wave; every lane gets it.
__device__ __forceinline__ void wave_best(float& v, int32_t& i) {
    dpp_best<dpp::kQuadXor1>(v, i);
    dpp_best<dpp::kQuadXor2>(v, i);
    dpp_best<dpp::kRowHalfMirror>(v, i);
    dpp_best<dpp::kRowMirror>(v, i);
    for (int off = 16; off < 64; off <<= 1) {
        const float ov = __shfl_xor(v, off, 64);
        const int32_t oi = __shfl_xor(i, off, 64);
        if (better(ov, oi, v, i)) {
            v = ov;
            i = oi;
        }
    }
}

// Best over the block (kBlock threads); every thread gets it.
__device__ __forceinline__ void block_best(float& v, int32_t& i) {
    __shared__ float sv[kBlock / 64];
    __shared__ int32_t si[kBlock / 64];
    wave_best(v, i);
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = v;
        si[threadIdx.x >> 6] = i;
    }
    __syncthreads();
    v = sv[0];
    i = si[0];
    for (int w = 1; w < kBlock / 64; ++w)
        if (better(sv[w], si[w], v, i)) {
            v = sv[w];
            i = si[w];
        }
    __syncthreads();
}

// grid (chunks, rows). A row of one chunk writes its result; otherwise partials [rows][chunks] (packed value, index).
__global__ __launch_bounds__(kBlock) void argmax_chunks(const float* __restrict__ x, float* __restrict__ values,
                                                        int32_t* __restrict__ indices, int64_t width, int chunks,
                                                        uint64_t* __restrict__ partials) {
    const int64_t row = blockIdx.y;
    const int chunk = blockIdx.x;
    const float* xr = x + row * width;
    const int64_t start = static_cast<int64_t>(chunk) * kChunk;
    const int64_t idx = start + threadIdx.x * 4;
    float bv = -INFINITY;
    int32_t bi = INT32_MAX;
    const bool vec_ok = (width % 4 == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0);
    if (vec_ok) {
        if (idx < width) {
            float f[4];
            unpack<F32>(ld128_nt(xr + idx), f);
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (better(f[k], static_cast<int32_t>(idx + k), bv, bi)) {
                    bv = f[k];
                    bi = static_cast<int32_t>(idx + k);
                }
        }
    } else {
        for (int k = 0; k < 4; ++k) {
            const int64_t j = idx + k;
            if (j < width) {
                const float v = xr[j];
                if (better(v, static_cast<int32_t>(j), bv, bi)) {
                    bv = v;
                    bi = static_cast<int32_t>(j);
                }
            }
        }
    }
    block_best(bv, bi);
    if (threadIdx.x != 0) return;
    if (chunks == 1) {
        if (bi == INT32_MAX) {  // no non-NaN value
            bi = 0;
            bv = xr[0];
        }
        values[row] = bv;
        indices[row] = bi;
    } else {
        partials[row * chunks + chunk] = pack_best(bv, bi);
    }
}

// grid (rows): the best of a row's partials.
__global__ __launch_bounds__(kBlock) void argmax_final(const float* __restrict__ x, float* __restrict__ values,
                                                       int32_t* __restrict__ indices, int64_t width, int chunks,
                                                       const uint64_t* __restrict__ partials) {
    const int64_t row = blockIdx.x;
    float bv = -INFINITY;
    int32_t bi = INT32_MAX;
    for (int c = threadIdx.x; c < chunks; c += kBlock) {
        const uint64_t b = partials[row * chunks + c];
        const float v = __uint_as_float(static_cast<uint32_t>(b));
        const int32_t i = static_cast<int32_t>(static_cast<uint32_t>(b >> 32));
        if (better(v, i, bv, bi)) {
            bv = v;
            bi = i;
        }
    }
    block_best(bv, bi);
    if (threadIdx.x == 0) {
        if (bi == INT32_MAX) {
            bi = 0;
            bv = x[row * width];
        }
        values[row] = bv;
        indices[row] = bi;
    }
}

// ---- k > 1 ----------------------------------------------------------------------------------------------------
//
// The order as one 64-bit word, larger = better: the high half maps the value's bits to unsigned order (+0 and -0 as
// one value), the low half is the complement of the index (the lower index larger). Distinct elements have distinct
// words, and 0 stands for "none" (NaN, or an element already taken): a real element's low half is at least 2^31.
__device__ __forceinline__ uint64_t order_word(float v, int64_t i) {
    if (v != v) return 0;
    const uint32_t b = __float_as_uint(v == 0.0f ? 0.0f : v);
    const uint32_t key = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return (static_cast<uint64_t>(key) << 32) | static_cast<uint32_t>(~static_cast<uint32_t>(i));
}
__device__ __forceinline__ int32_t word_index(uint64_t w) { return static_cast<int32_t>(~static_cast<uint32_t>(w)); }
__device__ __forceinline__ uint32_t word_bin(uint64_t w) { return static_cast<uint32_t>(w >> 53); }  // top 11 bits

template <int Ctrl>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
    const uint32_t lo = static_cast<uint32_t>(dpp_i<Ctrl>(static_cast<int>(v)));
    const uint32_t hi = static_cast<uint32_t>(dpp_i<Ctrl>(static_cast<int>(v >> 32)));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

// The largest word of the wave; every lane gets it.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    uint64_t o = dpp_u64<dpp::kQuadXor1>(v);
    v = o > v ? o : v;
    o = dpp_u64<dpp::kQuadXor2>(v);
    v = o > v ? o : v;
    o = dpp_u64<dpp::kRowHalfMirror>(v);
    v = o > v ? o : v;
    o = dpp_u64<dpp::kRowMirror>(v);
    v = o > v ? o : v;
    for (int off = 16; off < 64; off <<= 1) {
        o = __shfl_xor(v, off, 64);
        v = o > v ? o : v;
    }
    return v;
}

// Writes pick j of a row: the element named by word w, or (no element left: fewer than k non-NaN values) index 0 and
// x[0], as the k-pass selection reports it.
__device__ __forceinline__ void put_pick(const float* xr, float* values, int32_t* indices, int64_t at, uint64_t w) {
    const int32_t i = w == 0 ? 0 : word_index(w);
    values[at] = xr[i];  // the element's own bits (-0 stays -0)
    indices[at] = i;
}

// Narrow rows (width <= 64 P): a wave per row, the row's words in registers, lane l holding elements l + 64 p. A pick
// is the wave's largest word; the lane that owned it drops it and finds its next best.
template <int P>
__global__ __launch_bounds__(kBlock) void topk_wave_rows(const float* __restrict__ x, float* __restrict__ values,
                                                         int32_t* __restrict__ indices, int64_t rows, int64_t width,
                                                         int64_t k) {
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (kBlock / 64) + (threadIdx.x >> 6);
    if (row >= rows) return;  // whole waves leave together
    const float* xr = x + row * width;
    uint64_t w[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const int64_t i = lane + 64 * p;
        w[p] = i < width ? order_word(xr[i], i) : 0;
    }
    uint64_t best = 0;
#pragma unroll
    for (int p = 0; p < P; ++p) best = w[p] > best ? w[p] : best;
    for (int64_t j = 0; j < k; ++j) {
        const uint64_t top = wave_max_u64(best);
        if (lane == 0) put_pick(xr, values, indices, row * k + j, top);
        if (top == 0) continue;
        if (best == top) {  // the owner drops it
            best = 0;
#pragma unroll
            for (int p = 0; p < P; ++p) {
                w[p] = w[p] == top ? 0 : w[p];
                best = w[p] > best ? w[p] : best;
            }
        }
    }
}

// Wide rows: the k-th largest word's top 11 bits (its bin) from a histogram of the row, then every element of that
// bin or above compacted as a candidate -- usually a few hundred -- and those ranked. Per row in scratch: the bins,
// the candidate count, the candidates. A row whose candidates overflow (a crowded bin) or that holds fewer than k
// non-NaN values is selected by k passes over it instead (topk_passes), with the same result.
constexpr int kBins = 2048;
constexpr int kCap = 4096;
constexpr int kWideChunk = kBlock * 16;  // values per workgroup of the histogram and compaction passes
constexpr int64_t kWideMaxK = 1024;
constexpr size_t kRowScratch = (kBins + 64) * 4 + kCap * 8;  // bins, count (+ padding to 256 bytes), candidates

struct WideRow {
    uint32_t* bins;
    uint32_t* count;
    uint64_t* cand;
};
__device__ __forceinline__ WideRow wide_row(void* scratch, int64_t row) {
    char* base = static_cast<char*>(scratch) + row * kRowScratch;
    return {reinterpret_cast<uint32_t*>(base), reinterpret_cast<uint32_t*>(base) + kBins,
            reinterpret_cast<uint64_t*>(base + (kBins + 64) * 4)};
}

__global__ __launch_bounds__(kBlock) void topk_wide_clear(void* scratch) {
    const WideRow r = wide_row(scratch, blockIdx.x);
    for (int b = threadIdx.x; b < kBins; b += kBlock) r.bins[b] = 0;
    if (threadIdx.x == 0) *r.count = 0;
}

// The element words of this workgroup's chunk, 16 a thread (four 4-value groups kBlock apart: each load instruction
// covers consecutive values).
__device__ __forceinline__ void chunk_words(const float* xr, int64_t width, int64_t start, bool vec, uint64_t* w) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int64_t i0 = start + (static_cast<int64_t>(q) * kBlock + threadIdx.x) * 4;
        if (vec && i0 + 3 < width) {
            float f[4];
            unpack<F32>(ld128_nt(xr + i0), f);
#pragma unroll
            for (int e = 0; e < 4; ++e) w[4 * q + e] = order_word(f[e], i0 + e);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) w[4 * q + e] = i0 + e < width ? order_word(xr[i0 + e], i0 + e) : 0;
        }
    }
}

__global__ __launch_bounds__(kBlock) void topk_wide_hist(const float* __restrict__ x, int64_t width, bool vec,
                                                         void* scratch) {
    __shared__ uint32_t bins[kBins];
    for (int b = threadIdx.x; b < kBins; b += kBlock) bins[b] = 0;
    __syncthreads();
    const int64_t row = blockIdx.y;
    uint64_t w[16];
    chunk_words(x + row * width, width, static_cast<int64_t>(blockIdx.x) * kWideChunk, vec, w);
#pragma unroll
    for (int e = 0; e < 16; ++e)
        if (w[e] != 0) atomicAdd(&bins[word_bin(w[e])], 1u);
    __syncthreads();
    const WideRow r = wide_row(scratch, row);
    for (int b = threadIdx.x; b < kBins; b += kBlock)
        if (bins[b] != 0) atomicAdd(&r.bins[b], bins[b]);
}

// The bin of the k-th largest word: the largest b whose bins b .. top hold at least k elements (0 when the row holds
// fewer than k: then everything is a candidate, and the final pass sees too few or too many).
__device__ uint32_t threshold_bin(const uint32_t* gbins, int64_t k) {
    constexpr int PER = kBins / kBlock;  // bins a thread, counted from the top
    __shared__ uint32_t part[kBlock];
    __shared__ uint32_t found;
    const int t = threadIdx.x;
    uint32_t c[PER];
    uint32_t sum = 0;
#pragma unroll
    for (int q = 0; q < PER; ++q) {
        c[q] = gbins[kBins - 1 - (t * PER + q)];
        sum += c[q];
    }
    part[t] = sum;
    if (t == 0) found = 0;
    __syncthreads();
    // Exclusive prefix over the threads (a few thousand at most: serial over a wave, then per thread)
    uint64_t before = 0;
    for (int u = 0; u < t; ++u) before += part[u];
    if (before < static_cast<uint64_t>(k) && before + sum >= static_cast<uint64_t>(k)) {
        uint64_t acc = before;
        for (int q = 0; q < PER; ++q) {
            acc += c[q];
            if (acc >= static_cast<uint64_t>(k)) {
                found = static_cast<uint32_t>(kBins - 1 - (t * PER + q));
                break;
            }
        }
    }
    __syncthreads();
    return found;
}

__global__ __launch_bounds__(kBlock) void topk_wide_compact(const float* __restrict__ x, int64_t width, bool vec,
                                                            int64_t k, void* scratch) {
    const int64_t row = blockIdx.y;
    const WideRow r = wide_row(scratch, row);
    const uint32_t bin = threshold_bin(r.bins, k);
    uint64_t w[16];
    chunk_words(x + row * width, width, static_cast<int64_t>(blockIdx.x) * kWideChunk, vec, w);
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const bool keep = w[e] != 0 && word_bin(w[e]) >= bin;
        const uint64_t mask = __ballot(keep);
        if (mask == 0) continue;
        uint32_t base = 0;
        if (lane == __builtin_ctzll(mask)) base = atomicAdd(r.count, static_cast<uint32_t>(__popcll(mask)));
        base = __shfl(base, __builtin_ctzll(mask), 64);
        const uint32_t slot = base + static_cast<uint32_t>(__popcll(mask & ((uint64_t{1} << lane) - 1)));
        if (keep && slot < kCap) r.cand[slot] = w[e];
    }
}

// The k best of a row by k passes over it: pick j is the best element strictly after pick j - 1.
__device__ void topk_passes(const float* xr, float* values, int32_t* indices, int64_t row, int64_t width, int64_t k) {
    uint64_t prev = ~uint64_t{0};  // above every word
    for (int64_t j = 0; j < k; ++j) {
        uint64_t best = 0;
        for (int64_t c = threadIdx.x; c < width; c += kBlock) {
            const uint64_t w = order_word(xr[c], c);
            if (w < prev && w > best) best = w;
        }
        __shared__ uint64_t red[kBlock / 64];
        best = wave_max_u64(best);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
        __syncthreads();
        best = red[0];
        for (int q = 1; q < kBlock / 64; ++q) best = red[q] > best ? red[q] : best;
        __syncthreads();
        if (threadIdx.x == 0) put_pick(xr, values, indices, row * k + j, best);
        if (best != 0) prev = best;
    }
}

// One workgroup per row: the candidates ranked (each one's rank = how many candidates beat it) or, past 512 of
// them, bitonic-sorted in LDS; the fallback rows by passes.
__global__ __launch_bounds__(kBlock) void topk_wide_finish(const float* __restrict__ x, float* __restrict__ values,
                                                           int32_t* __restrict__ indices, int64_t width, int64_t k,
                                                           void* scratch) {
    __shared__ uint64_t cand[kCap];
    const int64_t row = blockIdx.x;
    const float* xr = x + row * width;
    const WideRow r = wide_row(scratch, row);
    const uint32_t n = *r.count;
    if (n > static_cast<uint32_t>(kCap) || n < static_cast<uint64_t>(k)) {
        topk_passes(xr, values, indices, row, width, k);
        return;
    }
    for (uint32_t i = threadIdx.x; i < n; i += kBlock) cand[i] = r.cand[i];
    __syncthreads();
    if (n <= 512) {
        for (uint32_t i = threadIdx.x; i < n; i += kBlock) {
            const uint64_t w = cand[i];
            uint32_t rank = 0;
            for (uint32_t j = 0; j < n; ++j) rank += cand[j] > w ? 1u : 0u;
            if (rank < k) put_pick(xr, values, indices, row * k + rank, w);
        }
        return;
    }
    uint32_t size = 1;
    while (size < n) size <<= 1;
    for (uint32_t i = n + threadIdx.x; i < size; i += kBlock) cand[i] = 0;
    __syncthreads();
    for (uint32_t len = 2; len <= size; len <<= 1) {
        for (uint32_t stride = len / 2; stride > 0; stride >>= 1) {
            for (uint32_t i = threadIdx.x; i < size / 2; i += kBlock) {
                const uint32_t lo = (i / stride) * 2 * stride + (i % stride);
                const uint32_t hi = lo + stride;
                const bool descending = (lo & len) == 0;  // the final order is descending
                const uint64_t a = cand[lo], b = cand[hi];
                if ((a < b) == descending) {
                    cand[lo] = b;
                    cand[hi] = a;
                }
            }
            __syncthreads();
        }
    }
    for (int64_t j = threadIdx.x; j < k; j += kBlock) put_pick(xr, values, indices, row * k + j, cand[j]);
}

// k passes by a workgroup per row (the widest k).
__global__ __launch_bounds__(kBlock) void topk_select(const float* __restrict__ x, float* __restrict__ values,
                                                      int32_t* __restrict__ indices, int64_t width, int64_t k) {
    topk_passes(x + static_cast<int64_t>(blockIdx.x) * width, values, indices, blockIdx.x, width, k);
}

bool wide_path(int64_t width, int64_t k) { return k > 1 && width > 64 * 64 && k <= kWideMaxK; }

int64_t argmax_chunks_of(int64_t width) { return (width + kChunk - 1) / kChunk; }

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace
}  // namespace xs_hip

using namespace xs_hip;

extern "C" {

size_t xs_hip_topk_scratch(int64_t rows, int64_t width, int64_t k) {
    if (rows <= 0 || width <= 0) return 0;
    if (wide_path(width, k)) return static_cast<size_t>(rows) * kRowScratch;
    if (k != 1) return 0;
    const int64_t chunks = argmax_chunks_of(width);
    if (chunks <= 1) return 0;
    return align_up(static_cast<size_t>(rows * chunks) * sizeof(uint64_t), 256);
}

int xs_hip_topk(void* stream, const float* x, float* values, int32_t* indices, int64_t rows, int64_t width, int64_t k,
                void* scratch) {
    if (rows < 0 || width <= 0 || k < 1 || k > width)
        return fail(XS_HIP_EINVAL, "xs_hip_topk: topk " + std::to_string(k) + " of " + std::to_string(rows) +
                                       " rows of " + std::to_string(width));
    if (width > INT32_MAX)
        return fail(XS_HIP_EUNSUPPORTED, "xs_hip_topk: rows wider than 2^31 - 1 have no i32 index");
    if (rows == 0) return XS_HIP_OK;
    if (x == nullptr || values == nullptr || indices == nullptr) return fail(XS_HIP_EINVAL, "xs_hip_topk: null buffer");
    const hipStream_t s = as_stream(stream);
    if (k == 1) {
        const int64_t chunks = argmax_chunks_of(width);
        if (rows > kMaxRows || chunks > INT32_MAX)
            return fail(XS_HIP_EUNSUPPORTED, "xs_hip_topk: more than 65535 rows in one call");
        uint64_t* partials = nullptr;
        if (chunks > 1) {
            if (scratch == nullptr)
                return fail(XS_HIP_EINVAL, "xs_hip_topk: argmax over rows of " + std::to_string(width) +
                                               " needs xs_hip_topk_scratch bytes of scratch");
            if (reinterpret_cast<uintptr_t>(scratch) % 8 != 0)
                return fail(XS_HIP_EINVAL, "xs_hip_topk: scratch must be 8-byte aligned");
            partials = static_cast<uint64_t*>(scratch);
        }
        argmax_chunks<<<dim3(static_cast<unsigned>(chunks), static_cast<unsigned>(rows)), kBlock, 0, s>>>(
            x, values, indices, width, static_cast<int>(chunks), partials);
        int rc = check_launch("xs_hip_topk");
        if (rc != XS_HIP_OK || chunks == 1) return rc;
        argmax_final<<<static_cast<unsigned>(rows), kBlock, 0, s>>>(x, values, indices, width, static_cast<int>(chunks),
                                                                     partials);
        return check_launch("xs_hip_topk");
    }
    if (rows > INT32_MAX / kBlock) return fail(XS_HIP_EUNSUPPORTED, "xs_hip_topk: too many rows");
    if (width <= 64 * 64) {
        const unsigned blocks = static_cast<unsigned>((rows + kBlock / 64 - 1) / (kBlock / 64));
        const int64_t p = (width + 63) / 64;
        if (p <= 1) topk_wave_rows<1><<<blocks, kBlock, 0, s>>>(x, values, indices, rows, width, k);
        else if (p <= 2) topk_wave_rows<2><<<blocks, kBlock, 0, s>>>(x, values, indices, rows, width, k);
        else if (p <= 4) topk_wave_rows<4><<<blocks, kBlock, 0, s>>>(x, values, indices, rows, width, k);
        else if (p <= 8) topk_wave_rows<8><<<blocks, kBlock, 0, s>>>(x, values, indices, rows, width, k);
        else if (p <= 16) topk_wave_rows<16><<<blocks, kBlock, 0, s>>>(x, values, indices, rows, width, k);
        else if (p <= 32) topk_wave_rows<32><<<blocks, kBlock, 0, s>>>(x, values, indices, rows, width, k);
        else topk_wave_rows<64><<<blocks, kBlock, 0, s>>>(x, values, indices, rows, width, k);
        return check_launch("xs_hip_topk");
    }
    if (!wide_path(width, k)) {  // k past kWideMaxK: passes
        topk_select<<<static_cast<unsigned>(rows), kBlock, 0, s>>>(x, values, indices, width, k);
        return check_launch("xs_hip_topk");
    }
    if (rows > kMaxRows) return fail(XS_HIP_EUNSUPPORTED, "xs_hip_topk: more than 65535 rows in one call");
    if (scratch == nullptr || reinterpret_cast<uintptr_t>(scratch) % 8 != 0)
        return fail(XS_HIP_EINVAL, "xs_hip_topk: top-" + std::to_string(k) + " of rows of " + std::to_string(width) +
                                       " needs xs_hip_topk_scratch bytes of 8-byte aligned scratch");
    const bool vec = width % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
    const dim3 grid(static_cast<unsigned>((width + kWideChunk - 1) / kWideChunk), static_cast<unsigned>(rows));
    topk_wide_clear<<<static_cast<unsigned>(rows), kBlock, 0, s>>>(scratch);
    topk_wide_hist<<<grid, kBlock, 0, s>>>(x, width, vec, scratch);
    topk_wide_compact<<<grid, kBlock, 0, s>>>(x, width, vec, k, scratch);
    topk_wide_finish<<<static_cast<unsigned>(rows), kBlock, 0, s>>>(x, values, indices, width, k, scratch);
    return check_launch("xs_hip_topk");
}

}  // extern "C"
