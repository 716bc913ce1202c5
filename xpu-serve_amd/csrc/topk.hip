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
// drafter's candidates): each 4096-value chunk keeps the words from the bin of its own k-th largest up (an LDS
// histogram of the order words' top 11 bits), and one workgroup per row ranks the kept words from the largest of those
// bins up -- a few hundred, typically; a row with crowded bins, or with fewer than k non-NaN values, is selected by k
// passes over it, with the same result.
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

// Best over the block (kBlock threads); every thread gets it. Once per launch: no barrier follows the reads.
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

// grid (rows): the best of a row's partials (a partial a thread: one round of loads; a single wave looping over
// them measured 0.3 us slower).
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
// x[0], as the k-pass selection reports it. The value comes back from the word's key, which maps float bits one to
// one except +0 and -0 (one key): only then, or with no element, is x read for the element's own bits.
__device__ __forceinline__ void put_pick(const float* xr, float* values, int32_t* indices, int64_t at, uint64_t w) {
    const int32_t i = w == 0 ? 0 : word_index(w);
    const uint32_t key = static_cast<uint32_t>(w >> 32);
    const uint32_t bits = (key & 0x80000000u) ? (key & 0x7FFFFFFFu) : ~key;
    values[at] = w == 0 || bits == 0 ? xr[i] : __uint_as_float(bits);
    indices[at] = i;
}

// Threads of a wave-per-row workgroup (64 measured 0.6% slower at 2048 rows of 128).
constexpr int kWaveRowsBlock = 256;

// Narrow rows (width <= 64 P): a wave per row, the row's words in registers, lane l holding elements l + 64 p. A pick
// is the wave's largest word; the lane that owned it drops it and finds its next best.
template <int P>
__global__ __launch_bounds__(kWaveRowsBlock) void topk_wave_rows(const float* __restrict__ x, float* __restrict__ values,
                                                                 int32_t* __restrict__ indices, int64_t rows,
                                                                 int64_t width, int64_t k) {
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (kWaveRowsBlock / 64) + (threadIdx.x >> 6);
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

// Wide rows: a workgroup per chunk of kWideChunk values computes a lower bound T on the chunk's k-th largest word and
// writes every word >= T (the chunk's candidates) to its slot in scratch, with T and their count. T is the k-th
// largest of the workgroup's per-thread maxima when there are at least k of those (k distinct words are >= it), else
// the k-th largest of all the chunk's words; either is found by an LDS histogram over the 11 bits just below the
// highest bit where the histogrammed words differ, so the words spread over the bins. The row's k-th largest word is
// at least every chunk's, so every word of the row's top k is at least G = max T and sits among its chunk's
// candidates. A workgroup per row gathers the candidates >= G into LDS and narrows them by more such histograms to the
// words from the k-th largest's bin up, then ranks those. A row whose chunk overflows its slot or whose gathered
// candidates overflow LDS (crowded values), or that holds fewer than k non-NaN values, is selected by k passes over
// it instead (topk_passes), with the same result. Every scratch word read is written earlier in the same call, so
// scratch needs no clearing.
constexpr int kBins = 2048;  // 11 bits
constexpr int kCap = 4096;   // candidates gathered in LDS
constexpr int kWideChunk = kBlock * 16;
constexpr int64_t kWideMaxK = 1024;
constexpr uint32_t kRankMax = 128;  // ranked directly; more are narrowed, or bitonic-sorted at the last bit
constexpr int kGatherUnroll = 8;    // chunks a wave reads at once

// Candidate slot per chunk: room for 4k words (at least 256, at most the chunk).
__host__ __device__ constexpr int64_t chunk_cap(int64_t k) {
    return k * 4 < 256 ? 256 : (k * 4 > kWideChunk ? kWideChunk : k * 4);
}
int64_t wide_chunks(int64_t width) { return (width + kWideChunk - 1) / kWideChunk; }
// Per row: a header {T, count} (16 bytes) per chunk, then the chunks' candidate slots.
constexpr size_t kHeaderBytes = 16;
__host__ __device__ constexpr size_t wide_row_bytes(int64_t chunks, int64_t k) {
    return static_cast<size_t>(chunks) * (kHeaderBytes + static_cast<size_t>(chunk_cap(k)) * 8);
}
struct ChunkHeader {
    uint64_t bound;   // candidates are the words >= bound
    uint32_t count;   // candidates, stored or not
    uint32_t top;     // the chunk's largest value key (0: no non-NaN value)
};

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

// Inclusive prefix sum over the block's threads (in thread order); every thread gets its own.
__device__ __forceinline__ uint32_t block_inclusive_scan(uint32_t v) {
    __shared__ uint32_t wsum[kBlock / 64];
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t o = __shfl_up(v, off, 64);
        v += lane >= off ? o : 0u;
    }
    if (lane == 63) wsum[threadIdx.x >> 6] = v;
    __syncthreads();
    for (int q = 0; q < static_cast<int>(threadIdx.x >> 6); ++q) v += wsum[q];
    __syncthreads();
    return v;
}

// The largest and smallest of the block's words v that are nonzero (hi = 0 when there are none); every thread gets
// them.
__device__ __forceinline__ void block_range(uint64_t hi_v, uint64_t lo_v, uint64_t& hi, uint64_t& lo) {
    __shared__ uint64_t his[kBlock / 64], los[kBlock / 64];
    hi_v = wave_max_u64(hi_v);
    lo_v = ~wave_max_u64(~lo_v);
    if ((threadIdx.x & 63) == 0) {
        his[threadIdx.x >> 6] = hi_v;
        los[threadIdx.x >> 6] = lo_v;
    }
    __syncthreads();
    hi = his[0];
    lo = los[0];
    for (int q = 1; q < kBlock / 64; ++q) {
        hi = his[q] > hi ? his[q] : hi;
        lo = los[q] < lo ? los[q] : lo;
    }
    __syncthreads();
}

// The bin of the k-th largest word counted in `bins`, or -1 when they hold fewer than k; *above gets the count of
// words in the bins above it.
__device__ int threshold_bin(const uint32_t* bins, int64_t k, uint32_t* above) {
    constexpr int PER = kBins / kBlock;  // bins a thread, counted from the top
    __shared__ int found;
    __shared__ uint32_t found_above;
    const int t = threadIdx.x;
    uint32_t c[PER];
    uint32_t sum = 0;
#pragma unroll
    for (int q = 0; q < PER; ++q) {
        c[q] = bins[kBins - 1 - (t * PER + q)];
        sum += c[q];
    }
    if (t == 0) {
        found = -1;
        found_above = 0;
    }
    const uint32_t incl = block_inclusive_scan(sum);  // its barriers also order `found`
    const uint64_t before = incl - sum;
    if (before < static_cast<uint64_t>(k) && incl >= static_cast<uint64_t>(k)) {
        uint64_t acc = before;
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            if (acc < static_cast<uint64_t>(k) && acc + c[q] >= static_cast<uint64_t>(k)) {
                found = kBins - 1 - (t * PER + q);
                found_above = static_cast<uint32_t>(acc);
            }
            acc += c[q];
        }
    }
    __syncthreads();
    *above = found_above;
    return found;
}

// The histogram window for words in [lo, hi] (hi != lo): they share every bit from `top` up; the window is the 11 (or
// fewer) bits below it.
struct Window {
    int top, bottom;
};
__device__ __forceinline__ Window window_of(uint64_t hi, uint64_t lo) {
    const int top = 64 - __builtin_clzll(hi ^ lo);
    return {top, top > 11 ? top - 11 : 0};
}
__device__ __forceinline__ uint32_t window_bin(uint64_t w, Window win) {
    return static_cast<uint32_t>(w >> win.bottom) & ((1u << (win.top - win.bottom)) - 1u);
}
// The smallest word with the shared bits of `like` from win.top up and bin b in the window.
__device__ __forceinline__ uint64_t window_floor(uint64_t like, Window win, uint32_t b) {
    const uint64_t shared = win.top >= 64 ? 0 : (like >> win.top) << win.top;
    return shared | (static_cast<uint64_t>(b) << win.bottom);
}

// Largest / smallest u32 over the wave; every lane gets it.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, static_cast<uint32_t>(dpp_i<dpp::kQuadXor1>(static_cast<int>(v))));
    v = max(v, static_cast<uint32_t>(dpp_i<dpp::kQuadXor2>(static_cast<int>(v))));
    v = max(v, static_cast<uint32_t>(dpp_i<dpp::kRowHalfMirror>(static_cast<int>(v))));
    v = max(v, static_cast<uint32_t>(dpp_i<dpp::kRowMirror>(static_cast<int>(v))));
    v = max(v, static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), 16, 64)));
    return max(v, static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), 32, 64)));
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) { return ~wave_max_u32(~v); }

// 32-bit windows over value keys (the high half of a word): the bits below the highest where hi and lo differ.
__device__ __forceinline__ Window window_of32(uint32_t hi, uint32_t lo) {
    const int top = 32 - __builtin_clz(hi ^ lo);
    return {top, top > 11 ? top - 11 : 0};
}
__device__ __forceinline__ uint32_t window_bin32(uint32_t key, Window win) {
    return (key >> win.bottom) & ((1u << (win.top - win.bottom)) - 1u);
}

// Each lane's exclusive prefix of c (0..31) over the wave, and the wave's total, from c's bit planes.
__device__ __forceinline__ uint32_t wave_exclusive_small(uint32_t c, uint32_t& total) {
    const int lane = threadIdx.x & 63;
    const uint64_t below = (uint64_t{1} << lane) - 1;
    uint32_t before = 0;
    total = 0;
#pragma unroll
    for (int bit = 0; bit < 5; ++bit) {
        const uint64_t plane = __ballot((c >> bit) & 1u);
        before += static_cast<uint32_t>(__popcll(plane & below)) << bit;
        total += static_cast<uint32_t>(__popcll(plane)) << bit;
    }
    return before;
}

// grid (chunks, rows): the chunk's bound, count and candidates. The bound is a value key (the high half of a word):
// every word with a key at or above it is a candidate.
__global__ __launch_bounds__(kBlock) void topk_wide_chunks(const float* __restrict__ x, int64_t width, bool vec,
                                                           int64_t k, void* scratch) {
    __shared__ uint32_t bins[kBins];
    __shared__ uint32_t wave_nz[kBlock / 64], wave_hi[kBlock / 64], wave_lo_max[kBlock / 64],
        wave_lo_all[kBlock / 64];
    __shared__ uint32_t n;
    for (int b = threadIdx.x; b < kBins; b += kBlock) bins[b] = 0;
    if (threadIdx.x == 0) n = 0;
    const int64_t row = blockIdx.y;
    const int64_t chunks = gridDim.x;
    const int64_t cap = chunk_cap(k);
    const int wave = threadIdx.x >> 6;
    uint64_t w[16];
    chunk_words(x + row * width, width, static_cast<int64_t>(blockIdx.x) * kWideChunk, vec, w);
    uint32_t m = 0, lo_all = ~0u;  // value keys: the thread's largest, the smallest of its non-NaN ones
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const uint32_t key = static_cast<uint32_t>(w[e] >> 32);
        m = key > m ? key : m;
        lo_all = key != 0 && key < lo_all ? key : lo_all;
    }
    {
        const uint32_t nz = static_cast<uint32_t>(__popcll(__ballot(m != 0)));
        const uint32_t hi = wave_max_u32(m);
        const uint32_t lo_max = wave_min_u32(m != 0 ? m : ~0u);
        const uint32_t lo_a = wave_min_u32(lo_all);
        if ((threadIdx.x & 63) == 0) {
            wave_nz[wave] = nz;
            wave_hi[wave] = hi;
            wave_lo_max[wave] = lo_max;
            wave_lo_all[wave] = lo_a;
        }
    }
    __syncthreads();
    uint32_t nz = 0, hi = 0, lo_max = ~0u, lo_a = ~0u;
#pragma unroll
    for (int q = 0; q < kBlock / 64; ++q) {
        nz += wave_nz[q];
        hi = max(hi, wave_hi[q]);
        lo_max = min(lo_max, wave_lo_max[q]);
        lo_a = min(lo_a, wave_lo_all[q]);
    }
    // The k-th largest per-thread maximum bounds the chunk's k-th largest when there are k maxima; else all words.
    const bool by_max = k <= kBlock && nz >= static_cast<uint64_t>(k);  // uniform
    const uint32_t lo = by_max ? lo_max : lo_a;
    // With one distinct key, every histogrammed word has it: the k maxima, or all the non-NaN words.
    uint32_t bound = hi != 0 && hi == lo ? hi : 0;  // 0: keep every non-NaN word
    if (hi != 0 && hi != lo) {  // uniform
        const Window win = window_of32(hi, lo);
        if (by_max) {
            if (m != 0) atomicAdd(&bins[window_bin32(m, win)], 1u);
        } else {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const uint32_t key = static_cast<uint32_t>(w[e] >> 32);
                if (key != 0) atomicAdd(&bins[window_bin32(key, win)], 1u);
            }
        }
        __syncthreads();
        uint32_t above;
        const int b = threshold_bin(bins, k, &above);
        if (b >= 0) bound = ((win.top >= 32 ? 0u : (hi >> win.top) << win.top)) | (static_cast<uint32_t>(b) << win.bottom);
    }
    uint32_t mine = 0;
#pragma unroll
    for (int e = 0; e < 16; ++e) mine += w[e] != 0 && static_cast<uint32_t>(w[e] >> 32) >= bound ? 1u : 0u;
    uint32_t wave_total;
    const uint32_t before = wave_exclusive_small(mine, wave_total);
    uint32_t base_at = 0;
    if ((threadIdx.x & 63) == 0 && wave_total != 0) base_at = atomicAdd(&n, wave_total);
    base_at = static_cast<uint32_t>(__shfl(static_cast<int>(base_at), 0, 64));
    char* base = static_cast<char*>(scratch) + row * wide_row_bytes(chunks, k);
    uint64_t* cand = reinterpret_cast<uint64_t*>(base + chunks * kHeaderBytes) + blockIdx.x * cap;
    uint32_t at = base_at + before;
#pragma unroll
    for (int e = 0; e < 16; ++e)
        if (w[e] != 0 && static_cast<uint32_t>(w[e] >> 32) >= bound) {
            if (at < cap) cand[at] = w[e];
            ++at;
        }
    __syncthreads();
    if (threadIdx.x == 0) {
        ChunkHeader h;
        h.bound = static_cast<uint64_t>(bound) << 32;
        h.count = n;
        h.top = hi;
        reinterpret_cast<ChunkHeader*>(base)[blockIdx.x] = h;
    }
}

// Appends the words with keep set to out[..cap) at the LDS counter n (one atomic per wave); n counts every kept word,
// stored or not.
__device__ __forceinline__ void append_kept(bool keep, uint64_t w, uint32_t* n, uint64_t* out, uint32_t cap) {
    const int lane = threadIdx.x & 63;
    const uint64_t mask = __ballot(keep);
    if (mask == 0) return;
    const int leader = __builtin_ctzll(mask);
    uint32_t base = 0;
    if (lane == leader) base = atomicAdd(n, static_cast<uint32_t>(__popcll(mask)));
    base = __shfl(base, leader, 64);
    const uint32_t slot = base + static_cast<uint32_t>(__popcll(mask & ((uint64_t{1} << lane) - 1)));
    if (keep && slot < cap) out[slot] = w;
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

// One workgroup per row; see the wide-row outline above. The candidates >= G end up in registers, kPerThread a
// thread: copied from their chunks' slots at prefix offsets when they all fit, else gathered from G up by a wave per
// chunk through LDS. The first narrowing level histograms their value keys over [G, the largest chunk top].
constexpr int kFlatChunks = kBins;  // chunk prefix sums held in LDS (rows up to 8M values)
constexpr int kPerThread = kCap / kBlock;

__global__ __launch_bounds__(kBlock) void topk_wide_finish(const float* __restrict__ x, float* __restrict__ values,
                                                           int32_t* __restrict__ indices, int64_t width, int64_t k,
                                                           int64_t chunks, const void* scratch) {
    __shared__ uint64_t kept[kWideMaxK];
    __shared__ uint64_t staging[kCap];
    __shared__ uint32_t prefix[kFlatChunks];
    __shared__ uint32_t bins[kBins];
    __shared__ uint32_t rank_of[kRankMax];
    __shared__ uint32_t n, nk;
    __shared__ uint64_t red_bound[kBlock / 64];
    __shared__ uint32_t red_over[kBlock / 64], red_top[kBlock / 64], red_total[2];
    const int64_t row = blockIdx.x;
    const float* xr = x + row * width;
    const int64_t cap = chunk_cap(k);
    const char* base = static_cast<const char*>(scratch) + row * wide_row_bytes(chunks, k);
    const ChunkHeader* hdr = reinterpret_cast<const ChunkHeader*>(base);
    const uint64_t* slots = reinterpret_cast<const uint64_t*>(base + chunks * kHeaderBytes);
    const bool flat = chunks <= kFlatChunks;
    // Headers: G, the largest top, overflow, and (flat) each thread's run of kFlatChunks / kBlock chunks' counts.
    constexpr int PER = kFlatChunks / kBlock;
    uint64_t g = 0;
    uint32_t over = 0, sum = 0, top = 0;
    uint32_t cnt[PER];
    for (int b = threadIdx.x; b < kBins; b += kBlock) bins[b] = 0;
    if (flat) {
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const int64_t c = static_cast<int64_t>(threadIdx.x) * PER + q;
            const ChunkHeader h = c < chunks ? hdr[c] : ChunkHeader{0, 0, 0};
            g = h.bound > g ? h.bound : g;
            top = h.top > top ? h.top : top;
            over |= h.count > static_cast<uint32_t>(cap) ? 1u : 0u;
            cnt[q] = h.count;
            sum += h.count;
        }
    } else {
        for (int64_t c = threadIdx.x; c < chunks; c += kBlock) {
            const ChunkHeader h = hdr[c];
            g = h.bound > g ? h.bound : g;
            top = h.top > top ? h.top : top;
            over |= h.count > static_cast<uint32_t>(cap) ? 1u : 0u;
        }
    }
    const uint32_t incl = block_inclusive_scan(sum);
    if (flat) {
        uint32_t at = incl - sum;
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            prefix[threadIdx.x * PER + q] = at;  // exclusive prefix of chunk threadIdx.x * PER + q
            at += cnt[q];
        }
    }
    g = wave_max_u64(g);
    top = wave_max_u32(top);
    for (int off = 1; off < 64; off <<= 1) over |= __shfl_xor(over, off, 64);
    if ((threadIdx.x & 63) == 0) {
        red_bound[threadIdx.x >> 6] = g;
        red_over[threadIdx.x >> 6] = over;
        red_top[threadIdx.x >> 6] = top;
    }
    if (threadIdx.x == kBlock - 1) red_total[0] = incl;
    if (threadIdx.x == 0) {
        n = 0;
        nk = 0;
    }
    __syncthreads();
    for (int q = 0; q < kBlock / 64; ++q) {
        g = red_bound[q] > g ? red_bound[q] : g;
        top = red_top[q] > top ? red_top[q] : top;
        over |= red_over[q];
    }
    if (over != 0) {  // uniform: a chunk lost candidates
        topk_passes(xr, values, indices, row, width, k);
        return;
    }
    const uint32_t g_key = static_cast<uint32_t>(g >> 32);
    // Level 0 window over value keys in [G, top] (none when they are one key).
    const bool level0 = top > g_key;
    const Window win0 = level0 ? window_of32(top, g_key) : Window{0, 0};
    uint64_t c[kPerThread];  // flat index threadIdx.x + kBlock q; 0 = none
    uint32_t total;
    if (flat && red_total[0] <= static_cast<uint32_t>(kCap)) {
        total = red_total[0];
        // Candidate i lives in the chunk whose prefix is the last <= i: one branch-free binary search per candidate,
        // all of a thread's searches stepping together.
        uint32_t at[kPerThread];
#pragma unroll
        for (int q = 0; q < kPerThread; ++q) at[q] = 0;
        // prefix[c] for c >= chunks holds the total, above every i: a probe past the last chunk (clamped into the
        // array) is never taken, and the reads need no guard, so they overlap.
        const uint32_t nchunks = static_cast<uint32_t>(chunks);
        for (uint32_t step = nchunks > 1 ? 1u << (31 - __builtin_clz(nchunks - 1)) : 0u; step != 0; step >>= 1) {
#pragma unroll
            for (int q = 0; q < kPerThread; ++q) {
                const uint32_t i = threadIdx.x + kBlock * q;
                const uint32_t next = at[q] + step;
                at[q] = prefix[min(next, static_cast<uint32_t>(kFlatChunks - 1))] <= i ? next : at[q];
            }
        }
#pragma unroll
        for (int q = 0; q < kPerThread; ++q) {
            const uint32_t i = threadIdx.x + kBlock * q;
            c[q] = i < total ? slots[static_cast<int64_t>(at[q]) * cap + (i - prefix[at[q]])] : 0;
        }
#pragma unroll
        for (int q = 0; q < kPerThread; ++q) c[q] = c[q] >= g ? c[q] : 0;
    } else {
        // A wave takes kGatherUnroll chunks at once, its lanes over their candidates, keeping those >= G.
        const int lane = threadIdx.x & 63;
        for (int64_t c0 = static_cast<int64_t>(threadIdx.x >> 6) * kGatherUnroll; c0 < chunks;
             c0 += kGatherUnroll * (kBlock / 64)) {
            uint32_t cn[kGatherUnroll];
            uint32_t most = 0;
#pragma unroll
            for (int u = 0; u < kGatherUnroll; ++u) {
                cn[u] = c0 + u < chunks ? hdr[c0 + u].count : 0u;
                most = cn[u] > most ? cn[u] : most;
            }
            for (uint32_t j0 = 0; j0 < most; j0 += 64) {
                const uint32_t j = j0 + lane;
                uint64_t w[kGatherUnroll];
#pragma unroll
                for (int u = 0; u < kGatherUnroll; ++u) w[u] = j < cn[u] ? slots[(c0 + u) * cap + j] : 0;
#pragma unroll
                for (int u = 0; u < kGatherUnroll; ++u)
                    append_kept(w[u] != 0 && w[u] >= g, w[u], &n, staging, kCap);
            }
        }
        __syncthreads();
        total = n;
        if (total > static_cast<uint32_t>(kCap)) {
            topk_passes(xr, values, indices, row, width, k);
            return;
        }
#pragma unroll
        for (int q = 0; q < kPerThread; ++q) {
            const uint32_t i = threadIdx.x + kBlock * q;
            c[q] = i < total ? staging[i] : 0;
        }
    }
    // Narrow: every word >= floor is a candidate of the top k, `left` of the top k are in [floor, ceil] (the words
    // still being split) and the rest above ceil; `count` words are >= floor (an over-estimate until a level ran).
    uint64_t floor = g, ceil = ~uint64_t{0};
    uint32_t left = static_cast<uint32_t>(k), count = total;
    bool too_few = false;
    if (level0) {
#pragma unroll
        for (int q = 0; q < kPerThread; ++q)
            if (c[q] != 0) atomicAdd(&bins[window_bin32(static_cast<uint32_t>(c[q] >> 32), win0)], 1u);
        __syncthreads();
        uint32_t above;
        const int b = threshold_bin(bins, left, &above);
        if (b < 0) {
            too_few = true;
        } else {
            const uint32_t shared = win0.top >= 32 ? 0u : (top >> win0.top) << win0.top;
            const uint32_t fk = shared | (static_cast<uint32_t>(b) << win0.bottom);
            const uint32_t ck = fk | ((1u << win0.bottom) - 1u);
            count = static_cast<uint32_t>(k) - left + above + bins[b];
            left -= above;
            floor = static_cast<uint64_t>(fk) << 32;
            ceil = (static_cast<uint64_t>(ck) << 32) | 0xFFFFFFFFull;
        }
        __syncthreads();  // bins read before they are cleared again
    }
    while (!too_few && count > kRankMax) {
        uint64_t hi = 0, lo = ~uint64_t{0};
        uint32_t inside = 0;
#pragma unroll
        for (int q = 0; q < kPerThread; ++q) {
            const bool in = c[q] != 0 && c[q] >= floor && c[q] <= ceil;
            hi = in && c[q] > hi ? c[q] : hi;
            lo = in && c[q] < lo ? c[q] : lo;
            inside += in ? 1u : 0u;
        }
        const uint32_t in_all = block_inclusive_scan(inside);
        if (threadIdx.x == kBlock - 1) red_total[1] = in_all;
        block_range(hi, lo, hi, lo);  // its barrier publishes red_total[1]
        if (red_total[1] < left) {  // fewer than k non-NaN values in the row
            too_few = true;
            break;
        }
        if (hi == lo) {  // one word left to split: it is the k-th
            floor = hi;
            count = static_cast<uint32_t>(k);
            break;
        }
        const Window win = window_of(hi, lo);
        for (int b = threadIdx.x; b < kBins; b += kBlock) bins[b] = 0;
        __syncthreads();
#pragma unroll
        for (int q = 0; q < kPerThread; ++q)
            if (c[q] != 0 && c[q] >= lo && c[q] <= hi) atomicAdd(&bins[window_bin(c[q], win)], 1u);
        __syncthreads();
        uint32_t above;
        const int b = threshold_bin(bins, left, &above);  // found: `left` words lie in [lo, hi]
        count = static_cast<uint32_t>(k) - left + above + bins[b];
        left -= above;
        floor = window_floor(hi, win, static_cast<uint32_t>(b));
        ceil = floor | ((uint64_t{1} << win.bottom) - 1);
        __syncthreads();  // bins read before the next level clears them
    }
    if (!too_few) {
        if (threadIdx.x < kRankMax) rank_of[threadIdx.x] = 0;
        uint32_t mine = 0;
#pragma unroll
        for (int q = 0; q < kPerThread; ++q) mine += c[q] != 0 && c[q] >= floor ? 1u : 0u;
        uint32_t wave_total;
        const uint32_t before = wave_exclusive_small(mine, wave_total);
        uint32_t at = 0;
        if ((threadIdx.x & 63) == 0 && wave_total != 0) at = atomicAdd(&nk, wave_total);
        at = static_cast<uint32_t>(__shfl(static_cast<int>(at), 0, 64)) + before;
#pragma unroll
        for (int q = 0; q < kPerThread; ++q)
            if (c[q] != 0 && c[q] >= floor) {
                if (at < kWideMaxK) kept[at] = c[q];
                ++at;
            }
        __syncthreads();
        too_few = nk < static_cast<uint32_t>(k);  // uniform
    }
    if (too_few) {
        topk_passes(xr, values, indices, row, width, k);
        return;
    }
    // The kept words: count <= kRankMax of them, ranked below, or (k > kRankMax) exactly k, sorted.
    const uint32_t m = nk;
    if (m > kRankMax) {
        uint32_t size = 1;
        while (size < m) size <<= 1;
        for (uint32_t i = m + threadIdx.x; i < size; i += kBlock) kept[i] = 0;
        __syncthreads();
        for (uint32_t len = 2; len <= size; len <<= 1) {
            for (uint32_t stride = len / 2; stride > 0; stride >>= 1) {
                for (uint32_t i = threadIdx.x; i < size / 2; i += kBlock) {
                    const uint32_t lo = (i / stride) * 2 * stride + (i % stride);
                    const uint32_t hi = lo + stride;
                    const bool descending = (lo & len) == 0;  // the final order is descending
                    const uint64_t a = kept[lo], b = kept[hi];
                    if ((a < b) == descending) {
                        kept[lo] = b;
                        kept[hi] = a;
                    }
                }
                __syncthreads();
            }
        }
        for (int64_t j = threadIdx.x; j < k; j += kBlock) put_pick(xr, values, indices, row * k + j, kept[j]);
        return;
    }
    // Rank: the waves split the comparisons of each kept word.
    const int lane = threadIdx.x & 63;
    const uint32_t part = threadIdx.x >> 6;
    const uint32_t j_begin = m * part / (kBlock / 64), j_end = m * (part + 1) / (kBlock / 64);
    for (uint32_t i = lane; i < m; i += 64) {
        const uint64_t w = kept[i];
        uint32_t r = 0;
#pragma unroll 8
        for (uint32_t j = j_begin; j < j_end; ++j) r += kept[j] > w ? 1u : 0u;
        if (r != 0) atomicAdd(&rank_of[i], r);
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < m; i += kBlock)
        if (rank_of[i] < k) put_pick(xr, values, indices, row * k + rank_of[i], kept[i]);
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

// ---- argmax in one launch --------------------------------------------------------------------------------------
//
// grid (chunks, rows) of kBlock threads; a workgroup reduces `span` values of its row from chunk * span, kBlock * VPT * 4
// at a time (plain loads: at a few KiB a workgroup the load latency is the cost, and the non-temporal form measured
// 0.3-0.4 us slower), to the largest order word (the order above: the lower index wins an exact tie, NaN is never
// picked). A row of one chunk (span = width) writes its result there. Otherwise each workgroup but the row's last
// chunk publishes its word into the row's slot of `sync` with one device-scope atomic store and exits; the row's last
// chunk -- the row's last workgroup to be dispatched, so every other chunk of its row is already running or done and
// none of them waits on anything -- polls the row's slots until all are published, takes the largest, writes the
// row's value and index, and returns the slots to zero. `sync` holds rows * chunks 64-bit words, zero at entry and at
// exit; a published word is never 0 (a chunk with no non-NaN value publishes 1, below every element's word, whose low
// half, the complement of an index below 2^31, is at least 2^31). Every access to it is a relaxed device-scope atomic,
// which this part keeps coherent across the XCDs' L2s without cache write-back or invalidation. (A ticket counter a
// workgroup takes at its start, as the split softmax does, measured 1 us slower here: 149 workgroups' atomics on one
// address queue up.)
constexpr int kArgMaxChunks = 256;
constexpr int kArgMaxSplitRows = 256;
constexpr int kArgmaxPolls = 1 << 24;  // the poller's bound: far past the time its row's other chunks take to finish

__device__ __forceinline__ uint64_t block_max_u64(uint64_t v) {
    __shared__ uint64_t sv[kBlock / 64];
    v = wave_max_u64(v);
    if ((threadIdx.x & 63) == 0) sv[threadIdx.x >> 6] = v;
    __syncthreads();
    v = sv[0];
    for (int w = 1; w < kBlock / 64; ++w) v = sv[w] > v ? sv[w] : v;
    return v;
}

template <int VPT>
__global__ __launch_bounds__(kBlock) void argmax_split(const float* __restrict__ x, float* __restrict__ values,
                                                       int32_t* __restrict__ indices, int64_t width, int chunks,
                                                       int64_t span, bool vec, uint64_t* __restrict__ sync) {
    const int64_t row = blockIdx.y;
    const int chunk = blockIdx.x;
    const float* xr = x + row * width;
    const int64_t begin = static_cast<int64_t>(chunk) * span;
    const int64_t end = begin + span < width ? begin + span : width;
    uint64_t best = 0;
    for (int64_t start = begin; start < end; start += kBlock * VPT * 4) {
        if (vec) {
            u32x4 raw[VPT];
#pragma unroll
            for (int k = 0; k < VPT; ++k) {
                const int64_t idx = start + static_cast<int64_t>(threadIdx.x + k * kBlock) * 4;
                if (idx < end) raw[k] = ld128(xr + idx);
            }
#pragma unroll
            for (int k = 0; k < VPT; ++k) {
                const int64_t idx = start + static_cast<int64_t>(threadIdx.x + k * kBlock) * 4;
                if (idx < end) {
                    float f[4];
                    unpack<F32>(raw[k], f);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint64_t w = order_word(f[i], idx + i);
                        best = w > best ? w : best;
                    }
                }
            }
        } else {
#pragma unroll
            for (int k = 0; k < VPT; ++k)
                for (int i = 0; i < 4; ++i) {
                    const int64_t j = start + static_cast<int64_t>(threadIdx.x + k * kBlock) * 4 + i;
                    if (j < end) {
                        const uint64_t w = order_word(xr[j], j);
                        best = w > best ? w : best;
                    }
                }
        }
    }
    best = block_max_u64(best);
    if (chunks == 1) {
        if (threadIdx.x == 0) put_pick(xr, values, indices, row, best);
        return;
    }
    uint64_t* slots = sync + row * chunks;
    if (chunk != chunks - 1) {
        if (threadIdx.x == 0)
            __hip_atomic_store(slots + chunk, best == 0 ? uint64_t{1} : best, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    if (threadIdx.x >= 64) return;
    const int lane = threadIdx.x;
    for (int it = 0; it < kArgmaxPolls; ++it) {
        uint64_t m = 0;
        bool all = true;
        for (int j = lane; j < chunks - 1; j += 64) {
            const uint64_t w = __hip_atomic_load(slots + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            all = all && w != 0;
            m = w > m ? w : m;
        }
        if (__all(all)) {
            m = wave_max_u64(m == 1 ? 0 : m);
            best = m > best ? m : best;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    if (lane == 0) put_pick(xr, values, indices, row, best);
    for (int j = lane; j < chunks - 1; j += 64)
        __hip_atomic_store(slots + j, uint64_t{0}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Launch shape of xs_hip_argmax: vectors a lane per pass (1, 2, 4 or 8) and chunks a row. Rows are split into chunks
// of kBlock * VPT * 4 values, the smallest VPT keeping the launch within about eight workgroups a CU (2048) and a row
// within kArgMaxChunks; 256 rows or more, or rows too wide for that, take one workgroup a row (chunks = 1).
struct ArgmaxShape {
    int vpt = 1;
    int64_t chunks = 1;
};

ArgmaxShape argmax_shape(int64_t rows, int64_t width) {
    if (rows < kArgMaxSplitRows) {
        for (int vpt = 1; vpt <= 8; vpt *= 2) {
            const int64_t chunk = static_cast<int64_t>(kBlock) * vpt * 4;
            const int64_t chunks = (width + chunk - 1) / chunk;
            if (chunks <= kArgMaxChunks && (rows * chunks <= 2048 || vpt == 8)) return {vpt, chunks};
        }
    }
    return {4, 1};
}

extern "C" {

size_t xs_hip_topk_scratch(int64_t rows, int64_t width, int64_t k) {
    if (rows <= 0 || width <= 0) return 0;
    if (wide_path(width, k)) return static_cast<size_t>(rows) * wide_row_bytes(wide_chunks(width), k);
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
        const unsigned blocks = static_cast<unsigned>((rows + kWaveRowsBlock / 64 - 1) / (kWaveRowsBlock / 64));
        const int64_t p = (width + 63) / 64;
        if (p <= 1) topk_wave_rows<1><<<blocks, kWaveRowsBlock, 0, s>>>(x, values, indices, rows, width, k);
        else if (p <= 2) topk_wave_rows<2><<<blocks, kWaveRowsBlock, 0, s>>>(x, values, indices, rows, width, k);
        else if (p <= 4) topk_wave_rows<4><<<blocks, kWaveRowsBlock, 0, s>>>(x, values, indices, rows, width, k);
        else if (p <= 8) topk_wave_rows<8><<<blocks, kWaveRowsBlock, 0, s>>>(x, values, indices, rows, width, k);
        else if (p <= 16) topk_wave_rows<16><<<blocks, kWaveRowsBlock, 0, s>>>(x, values, indices, rows, width, k);
        else if (p <= 32) topk_wave_rows<32><<<blocks, kWaveRowsBlock, 0, s>>>(x, values, indices, rows, width, k);
        else topk_wave_rows<64><<<blocks, kWaveRowsBlock, 0, s>>>(x, values, indices, rows, width, k);
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
    const int64_t chunks = wide_chunks(width);
    if (chunks > INT32_MAX) return fail(XS_HIP_EUNSUPPORTED, "xs_hip_topk: row too wide");
    topk_wide_chunks<<<dim3(static_cast<unsigned>(chunks), static_cast<unsigned>(rows)), kBlock, 0, s>>>(x, width, vec,
                                                                                                        k, scratch);
    topk_wide_finish<<<static_cast<unsigned>(rows), kBlock, 0, s>>>(x, values, indices, width, k, chunks, scratch);
    return check_launch("xs_hip_topk");
}

size_t xs_hip_argmax_scratch(int64_t rows, int64_t width) {
    if (rows <= 0 || width <= 0) return 0;
    const int64_t chunks = argmax_shape(rows, width).chunks;
    return chunks <= 1 ? 0 : align_up(static_cast<size_t>(rows * chunks) * sizeof(uint64_t), 256);
}

int xs_hip_argmax(void* stream, const float* x, float* values, int32_t* indices, int64_t rows, int64_t width,
                  void* scratch) {
    if (rows < 0 || width <= 0)
        return fail(XS_HIP_EINVAL, "xs_hip_argmax: " + std::to_string(rows) + " rows of " + std::to_string(width));
    if (width > INT32_MAX)
        return fail(XS_HIP_EUNSUPPORTED, "xs_hip_argmax: rows wider than 2^31 - 1 have no i32 index");
    if (rows == 0) return XS_HIP_OK;
    if (x == nullptr || values == nullptr || indices == nullptr)
        return fail(XS_HIP_EINVAL, "xs_hip_argmax: null buffer");
    if (rows > kMaxRows) return fail(XS_HIP_EUNSUPPORTED, "xs_hip_argmax: more than 65535 rows in one call");
    const ArgmaxShape sh = argmax_shape(rows, width);
    if (sh.chunks > 1 && (scratch == nullptr || reinterpret_cast<uintptr_t>(scratch) % 8 != 0))
        return fail(XS_HIP_EINVAL, "xs_hip_argmax: rows of " + std::to_string(width) +
                                       " need xs_hip_argmax_scratch bytes of zero-filled, 8-byte aligned scratch");
    const bool vec = width % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
    const int64_t span = sh.chunks > 1 ? static_cast<int64_t>(kBlock) * sh.vpt * 4 : width;
    const dim3 grid(static_cast<unsigned>(sh.chunks), static_cast<unsigned>(rows));
    const hipStream_t s = as_stream(stream);
    auto* sync = static_cast<uint64_t*>(scratch);
    const int c = static_cast<int>(sh.chunks);
    switch (sh.vpt) {
        case 1: argmax_split<1><<<grid, kBlock, 0, s>>>(x, values, indices, width, c, span, vec, sync); break;
        case 2: argmax_split<2><<<grid, kBlock, 0, s>>>(x, values, indices, width, c, span, vec, sync); break;
        case 4: argmax_split<4><<<grid, kBlock, 0, s>>>(x, values, indices, width, c, span, vec, sync); break;
        default: argmax_split<8><<<grid, kBlock, 0, s>>>(x, values, indices, width, c, span, vec, sync); break;
    }
    return check_launch("xs_hip_argmax");
}

}  // extern "C"
