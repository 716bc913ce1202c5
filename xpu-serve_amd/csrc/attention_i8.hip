// Decode attention for gfx950 over the KV caches: the int8 reader of the codes and scales xs_hip_quantize_kv writes
// (this header), and further down one reader for the Float format's rows and the TurboQuant caches.
//
// Semantics: cpu_ref::attention / attend_one (reference src/backend/cpu_ref/ops.cpp:113-156, 535-594) over the
// values the int8 cache stores, fl32(code * scale) (quant::round_trip_kv_i8, src/quant/quant.cpp:269-277; the CPU
// cache holds exactly those values, cpu_backend.cpp:529-544): for query head h of token t at position
// pos = kv_len - tokens + t, over keys [first, last] (causal: last = pos; a sliding window of w keeps
// [pos - w + 1, pos + w - 1]; otherwise every key), s_j = scale * q . k_j (softcap: cap * tanh(s / cap)),
// p_j = exp(s_j - max) / sum, out = sum p_j v_j. Grouped-query: query head h reads KV head h / (q_heads / kv_heads).
// Launcher replaced: sycl_be::attention_rows_quantized with attention_combine (src/backend/sycl/sycl_kernels.h:
// 238-240), I8 rows (sycl_kv_rows.h:37-69).
//
// Layout: one workgroup per (token, group of KV heads, key split), one wave per KV head of the group (waves_for and
// the kernel's comment give the shapes); each wave takes tiles of 64 keys of the split, loads the next tile's key and
// value rows while it works on the current one, and runs one online softmax for the G query heads of its KV head.
// Both products (scores and the weighted sum) run on the int8 matrix cores with exact integer dot products. With one
// split the workgroup writes the output; with several it writes partial sums with their (max, sum of exponentials)
// that a second launch merges (flash decoding).
//
// Accuracy: f32 accumulation where cpu-ref accumulates in f64, the key scale applied to the dot product rather than
// to each product, and q and the softmax weights taken as 23-bit integers (relative 2^-23 of the head's max |q| and of
// the tile's largest weight) -- within the reference's own device tolerance for a quantized cache
// (tests/unit/backend/device_attention.cpp:23-27).
#include <cmath>
#include <type_traits>

#include <mutex>

#include "common.h"
#include "kv_turbo.h"

namespace xs_hip {
namespace {

struct AttnArgs {
    const float* q;       // [T, Hq, D]
    const int8_t* kc;     // [N, Hkv, D] key codes
    const float* ks;      // [N, Hkv] key scales
    const int8_t* vc;     // [N, Hkv, D] value codes
    const float* vs;      // [N, Hkv] value scales
    float* out;           // [T, Hq, D], or null when `part` is written
    float* part;          // sums [T * Hq * split, D], then (max, sum) [T * Hq * split, 2]; or null
    int64_t tokens, q_heads, kv_heads, head_dim, kv_len, window;
    float scale, softcap;
    int causal, split;
    int hg;  // KV heads a workgroup (8, 4, 2 or 1)
    // Or the key count read from device memory when the kernel runs (a step replayed from a captured graph), clamped
    // to [0, kv_len]: kv_len is then the cache's capacity.
    const int64_t* kv_len_dev = nullptr;
};

// The keys the cache holds for this launch.
__device__ __forceinline__ int64_t keys_of(const AttnArgs& a) {
    if (a.kv_len_dev == nullptr) return a.kv_len;
    const int64_t n = a.kv_len_dev[0];
    return n < 0 ? 0 : (n > a.kv_len ? a.kv_len : n);
}

// The key range [first, last] of query token t over n keys (cpu_ref::attention, ops.cpp:565-575 without blocks and
// anchors).
__device__ __forceinline__ void key_range(const AttnArgs& a, int64_t n, int64_t t, int64_t& first, int64_t& last) {
    const int64_t pos = n - a.tokens + t;
    first = a.window > 0 ? (pos - a.window + 1 > 0 ? pos - a.window + 1 : 0) : 0;
    last = a.causal ? pos : n - 1;
    if (a.window > 0 && pos + a.window - 1 < last) last = pos + a.window - 1;
}

// Waves a workgroup: eight (two a SIMD) where a wave's registers fit in 256, four for the wider cases (head_dim 256,
// or five to eight query heads a KV head at head_dim 128).
constexpr int waves_for(int G, int D) { return D * ((G + 3) / 4) <= 128 ? 8 : 4; }
constexpr int kMaxWaves = 8;

// Buffer resources over raw bytes (word 3: 32-bit data format, no swizzle); loads beyond num_records return zeros.
constexpr int kBufferFlags = 0x00020000;
constexpr int kBufferNt = 2;  // the non-temporal hint of a buffer load
constexpr int kTile = 64;    // keys a wave works on at once (at most 64: one a lane for the scales)

// Merges (m, l, acc) of another key set into this one: the online-softmax combine.
template <int N>
__device__ __forceinline__ void merge(float& m, float& l, float* acc, float mo, float lo, const float* acco) {
    const float mm = fmaxf(m, mo);
    const float ca = m == -INFINITY ? 0.0f : __expf(m - mm);  // an empty side (max -inf) contributes nothing
    const float cb = mo == -INFINITY ? 0.0f : __expf(mo - mm);
    l = l * ca + lo * cb;
#pragma unroll
    for (int i = 0; i < N; ++i) acc[i] = acc[i] * ca + acco[i] * cb;
    m = mm;
}

__device__ __forceinline__ float byte_f32(uint32_t w, int k) {
    return static_cast<float>(static_cast<int8_t>((w >> (8 * k)) & 0xffu));
}

typedef int i32x4 __attribute__((ext_vector_type(4)));

typedef int i32x2 __attribute__((ext_vector_type(2)));

// Reads 8 bytes a lane from LDS with the transpose of ds_read_b64_tr_b8: within each group of 16 lanes, with C_j the
// 8 bytes at lane j's address, lane i receives byte i % 8 of C_{2k + i / 8} as its byte k (k < 8). Lane j pointing at
// row base + j / 2, column col + 8 (j % 2) of a row-major byte tile thus gives lane i column col + i of rows
// base .. base + 7: a 16-column by 8-row block, transposed.
__device__ __forceinline__ i32x2 lds_read_tr8(const uint8_t* p) {
    // p points into LDS: the C cast converts the generic address to the LDS address space the builtin takes.
    return __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) i32x2*)(p));
}

// Byte d (d < 3) of the balanced base-256 digits of an integer |Q| < 2^23 (Q = hi 65536 + mid 256 + lo, each digit in
// [-128, 127]); the signed byte of digit d is byte d of Q + bias_d, bias = {0, 128, 32896}: with lo + 128 in
// [0, 255], (Q + 128) >> 8 = hi 256 + mid, and (Q + 32896) >> 16 = hi.
__device__ __forceinline__ int digit_bias(int d) { return d == 0 ? 0 : d == 1 ? 128 : 32896; }

// Packs byte `d` of each of four words into one (v_perm_b32; `sel` = d * 0x01010101 selects byte d of every source).
__device__ __forceinline__ int pack_bytes(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3, uint32_t d) {
    // v_perm_b32(s0, s1, sel): byte selector k picks byte k of {s1 (bytes 0-3), s0 (bytes 4-7)}.
    const uint32_t lo = __builtin_amdgcn_perm(w1, w0, 0x0c0c0400u + d * 0x0101u);  // [w0.d, w1.d, 0, 0]
    const uint32_t hi = __builtin_amdgcn_perm(w3, w2, 0x04000c0cu + d * 0x01010000u);  // [0, 0, w2.d, w3.d]
    return static_cast<int>(lo | hi);
}

// G query heads per KV head, D head_dim (64, 128 or 256), CAP: a softcap on the scores.
//
// A workgroup of W waves (waves_for) takes one split of the keys of HG KV heads (HG = the largest power of two up to
// W dividing kv_heads): wave w works on KV head w % HG and takes the split's tiles of 64 keys w / HG,
// w / HG + W / HG, ... With HG = 8 the eight waves read the eight heads' rows of the same keys -- contiguous
// [keys, heads, head_dim] spans -- together.
// Each wave keeps the next tile's codes and scales loading into registers while it works on the current one.
//
// Both products run on the int8 matrix cores (v_mfma_i32_16x16x64_i8: A [16 x 64] x B [64 x 16], i32 results), with
// the f32 operand written as three balanced base-256 int8 digits of an integer, so every product is exact:
//  - scores: S^T [16 rows, 16 keys] = digits of q [16 rows, 64 dims] x key codes^T [64 dims, 16 keys], one 64-dim
//    chunk at a time. Row 4 g + d holds digit d of head g (q / qs rounded, qs = max |q| / 2^22; row 4 g + 3 is zero),
//    four heads a step. Lane l reads 16 codes of key l % 16, dims 16 (l / 16) .., from the staged key tile and
//    receives rows 4 (l / 16) + r: the three digit sums of head l / 16 and key l % 16, combined in f32.
//  - the weighted sum: O^T [16 dims, 16 cols] = value codes^T [16 dims, 64 keys] x weight digits [64 keys, 16 cols],
//    column 4 g + d holding digit d of W = p v_scale / ws for head g (ws = the tile's max p v_scale / 2^22).
//    The value tile is staged in LDS and read transposed (lds_read_tr8); lane l receives dims 4 (l / 16) + r of
//    column l % 16, which it accumulates in f32 times ws 256^d. The digit columns of a head add up at the end.
template <int G, int D, bool CAP>
__global__ __launch_bounds__(64 * waves_for(G, D)) void attention_i8_rows(AttnArgs a) {
    constexpr int kWaves = waves_for(G, D);
    constexpr int NG = (G + 3) / 4;        // groups of four heads: one matrix-core step each
    constexpr int KC = D / 64;             // 64-dim chunks of a key row: the K of one score step
    constexpr int KB = kTile / 16;         // 16-key blocks of a tile: the N of one score step
    constexpr int DB = D / 16;             // 16-dim blocks of a value row: the M of one weighted-sum step
    constexpr int VROW = D + 16;           // LDS bytes a staged value row (16 bytes of padding: the eight rows one
                                           // transposed read covers start on distinct banks)
    constexpr int VLPR = D / 16;           // lanes a value row with 16-byte loads
    constexpr int VRPI = 64 / VLPR;        // value rows one load instruction covers
    constexpr int VI = kTile / VRPI;       // value load instructions a tile
    constexpr int VT = kTile * VROW;       // bytes of a wave's value tile, and of its key tile
    constexpr int PT = NG * 4 * kTile * 4; // bytes of a wave's weight tile: W [NG * 4 heads][kTile keys]
    constexpr int WAVE_LDS = 2 * VT + PT + 2 * kTile * 4;
    constexpr int MROW = D + 2;            // a merge row: D sums, max, sum
    static_assert(G >= 1 && G <= 8, "one or two groups of four heads");
    static_assert(kTile == 64, "a weighted-sum step takes the 64 keys of a tile");
    static_assert(kWaves * G * MROW * 4 <= kWaves * WAVE_LDS, "the merge rows fit in the tiles' LDS");
    __shared__ __align__(16) uint8_t lds[kWaves * WAVE_LDS];

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int c16 = lane & 15;  // the key (score step) or column (weighted-sum step) of this lane
    const int kq = lane >> 4;   // its 16-dim / 16-key / 4-row group
    const int hg = a.hg;
    const int np = kWaves / hg;  // waves a KV head
    const int phase = wave / hg;
    const int64_t groups = a.kv_heads / hg;
    const int64_t t = blockIdx.y / groups;
    const int64_t kvh = (blockIdx.y - t * groups) * hg + wave % hg;
    const int s = blockIdx.x;

    uint8_t* const vt = lds + wave * WAVE_LDS;
    uint8_t* const kt = vt + VT;
    float* const ptile = reinterpret_cast<float*>(kt + VT);  // [NG * 4][kTile]
    float* const kscale = ptile + NG * 4 * kTile;            // [kTile]
    float* const vscale = kscale + kTile;                    // [kTile]

    int64_t first, last;
    key_range(a, keys_of(a), t, first, last);
    const int64_t len = last >= first ? last - first + 1 : 0;
    const int64_t per = (len + a.split - 1) / a.split;
    const int64_t k0 = first + s * per;
    int64_t k1 = k0 + per - 1;
    if (k1 > last) k1 = last;
    const int64_t span = k1 >= k0 ? k1 - k0 + 1 : 0;
    const int64_t tiles = (span + kTile - 1) / kTile;

    // Loads of one tile into registers: key codes in the score step's B layout, value codes (for LDS), this lane's
    // key's scales. Buffer loads: the tile's rows of this KV head are addressed from one uniform base with 32-bit lane
    // offsets, and the buffer's extent ends at key k1, so the rows of keys past the split's last read as zeros (their
    // weights are 0).
    u32x4 kw[VI];
    u32x4 vw[VI];
    float ksv = 0.0f, vsv = 0.0f;
    const int64_t rstride = a.kv_heads * D;  // bytes from one key's row to the next of the same KV head
    const uint32_t voff = static_cast<uint32_t>((lane / VLPR) * rstride + (lane % VLPR) * 16);
    const uint32_t soff = static_cast<uint32_t>(lane * a.kv_heads * 4);
    auto load_tile = [&](int64_t j0) {
        const int64_t row0 = j0 * a.kv_heads + kvh;  // (key j0, this KV head)
        const int64_t rows_left = k1 - j0;           // keys after j0 within the split
        // Extents past 2^31 - 1 bytes are clamped there: the tile's offsets stay below 64 rows.
        const int nk = static_cast<int>(rows_left * rstride + D < 0x7fffffff ? rows_left * rstride + D : 0x7fffffff);
        const int64_t ns64 = (rows_left * a.kv_heads + 1) * 4;
        const int ns = static_cast<int>(ns64 < 0x7fffffff ? ns64 : 0x7fffffff);
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<int8_t*>(a.kc + row0 * D), 0, nk, kBufferFlags);
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<int8_t*>(a.vc + row0 * D), 0, nk, kBufferFlags);
        const __amdgpu_buffer_rsrc_t rks = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(a.ks + row0), 0, ns, kBufferFlags);
        const __amdgpu_buffer_rsrc_t rvs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(a.vs + row0), 0, ns, kBufferFlags);
#pragma unroll
        for (int i = 0; i < VI; ++i)
            kw[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  rk, static_cast<int>(voff + i * VRPI * rstride), 0, kBufferNt));
#pragma unroll
        for (int i = 0; i < VI; ++i)
            vw[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  rv, static_cast<int>(voff + i * VRPI * rstride), 0, kBufferNt));
        ksv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rks, static_cast<int>(soff), 0, 0));
        vsv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rvs, static_cast<int>(soff), 0, 0));
    };

    // q as digit rows (the score step's A operand): lane l holds digit l % 4 of head (l % 16) / 4 + 4 ng over dims
    // 64 c + 16 (l / 16) ..; score_scale[ng] is qs * scale of head l / 16 + 4 ng, the head of this lane's scores.
    i32x4 qa[NG][KC];
    float score_scale[NG];
    {
        const int dq = c16 & 3;
        u32x4 raw[NG][KC][4];
#pragma unroll
        for (int ng = 0; ng < NG; ++ng) {
            const int g = (c16 >> 2) + 4 * ng;
            const float* q = a.q + (t * a.q_heads + kvh * G + (g < G ? g : G - 1)) * D;
#pragma unroll
            for (int c = 0; c < KC; ++c) {
#pragma unroll
                for (int i = 0; i < 4; ++i) raw[ng][c][i] = ld128(q + c * 64 + kq * 16 + 4 * i);
            }
        }
        // The first tile's loads go out behind q's, to be in flight while the digits are made.
        if (phase < tiles) load_tile(k0 + phase * kTile);
#pragma unroll
        for (int ng = 0; ng < NG; ++ng) {
            float mx = 0.0f;
#pragma unroll
            for (int c = 0; c < KC; ++c) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) mx = fmaxf(mx, fabsf(__uint_as_float(raw[ng][c][i][e])));
                }
            }
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));  // max |q| of head (l % 16) / 4 + 4 ng over all its dims
            const float inv = mx > 0.0f ? 4194304.0f / mx : 0.0f;
            const bool live = dq < 3 && (c16 >> 2) + 4 * ng < G;
            const int bias = digit_bias(dq);
#pragma unroll
            for (int c = 0; c < KC; ++c) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    uint32_t w[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        w[e] = static_cast<uint32_t>(static_cast<int>(rintf(__uint_as_float(raw[ng][c][i][e]) * inv)) +
                                                     bias);
                    qa[ng][c][i] = live ? pack_bytes(w[0], w[1], w[2], w[3], static_cast<uint32_t>(dq)) : 0;
                }
            }
            score_scale[ng] = __shfl(mx, 4 * kq, 64) * (1.0f / 4194304.0f) * a.scale;
        }
    }

    // Running state. Score lanes (row kq) follow head kq + 4 ng: its running max m and their share of its sum of
    // exponentials. Weighted-sum lanes hold column c16 = (head (c16 / 4) + 4 ng, digit c16 % 4), dims
    // 16 db + 4 kq + r.
    float m[NG], lsum[NG];
    float facc[NG][DB][4];
#pragma unroll
    for (int ng = 0; ng < NG; ++ng) {
        m[ng] = -INFINITY;
        lsum[ng] = 0.0f;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
            for (int r = 0; r < 4; ++r) facc[ng][db][r] = 0.0f;
        }
    }
    const uint32_t dcol = static_cast<uint32_t>(c16 & 3);
    const int wbias = digit_bias(static_cast<int>(dcol));
    const float dscale = dcol == 0 ? 1.0f : dcol == 1 ? 256.0f : dcol == 2 ? 65536.0f : 0.0f;

    // The waves run independently: each touches only its own LDS, whose writes and reads are ordered within the
    // wave (wave_sync).
    auto wave_sync = [] {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    for (int64_t tile = phase; tile < tiles; tile += np) {
        const int64_t j0 = k0 + tile * kTile;  // keys j0 .. j0 + 63 (those past k1 clamped to it, weights 0)
        // Stage: key and value codes and the scales to LDS.
#pragma unroll
        for (int i = 0; i < VI; ++i) {
            const int at = (i * VRPI + lane / VLPR) * VROW + (lane % VLPR) * 16;
            *reinterpret_cast<u32x4*>(kt + at) = kw[i];
            *reinterpret_cast<u32x4*>(vt + at) = vw[i];
        }
        kscale[lane] = ksv;
        vscale[lane] = vsv;
        wave_sync();

        // Scores.
        i32x4 sr[NG][KB];
#pragma unroll
        for (int ng = 0; ng < NG; ++ng) {
#pragma unroll
            for (int b = 0; b < KB; ++b) {
                i32x4 acc = {0, 0, 0, 0};
#pragma unroll
                for (int c = 0; c < KC; ++c) {
                    // key 16 b + c16, dims 64 c + 16 kq ..: 16 bytes of its staged row (the rows' 16-byte padding
                    // spreads the 16 rows one read covers over all banks)
                    const i32x4 kb = *reinterpret_cast<const i32x4*>(kt + (b * 16 + c16) * VROW + c * 64 + kq * 16);
                    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa[ng][c], kb, acc, 0, 0, 0);
                }
                sr[ng][b] = acc;
            }
        }
        // The next tile's loads, into the registers just staged (uniform branch).
        if (tile + np < tiles) load_tile(j0 + np * kTile);

        float ksc[KB];
#pragma unroll
        for (int b = 0; b < KB; ++b) ksc[b] = kscale[b * 16 + c16];
        float sc[NG][KB];
        float mt[NG];
        bool moved = false;
#pragma unroll
        for (int ng = 0; ng < NG; ++ng) {
            const bool head_ok = kq + 4 * ng < G;
            mt[ng] = -INFINITY;
#pragma unroll
            for (int b = 0; b < KB; ++b) {
                const float dot = fmaf(static_cast<float>(sr[ng][b][2]), 65536.0f,
                                       fmaf(static_cast<float>(sr[ng][b][1]), 256.0f, static_cast<float>(sr[ng][b][0])));
                float x = dot * (score_scale[ng] * ksc[b]);
                if constexpr (CAP) x = a.softcap * tanhf(x / a.softcap);
                const bool valid = head_ok && j0 + b * 16 + c16 <= k1;
                sc[ng][b] = valid ? x : -INFINITY;
                mt[ng] = fmaxf(mt[ng], sc[ng][b]);
            }
            mt[ng] = group_reduce<16, OpMax>(mt[ng]);  // the tile's max of head kq + 4 ng
            moved |= mt[ng] > m[ng];
        }
        // A larger max for some head (uniform branch): rescale its sum and its columns' sums by exp(old - new).
        if (__builtin_amdgcn_ballot_w64(moved) != 0) {
#pragma unroll
            for (int ng = 0; ng < NG; ++ng) {
                const float mn = fmaxf(m[ng], mt[ng]);
                const float c = m[ng] == -INFINITY ? 0.0f : __expf(m[ng] - mn);
                lsum[ng] *= c;
                m[ng] = mn;
                const float cc = __shfl(c, 16 * (c16 >> 2), 64);  // the factor of this lane's column head
#pragma unroll
                for (int db = 0; db < DB; ++db) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) facc[ng][db][r] *= cc;
                }
            }
        }
        // p = exp(s - max) and the weights w = p v_scale; as integers W = w / ws, ws = the tile's max w of the head
        // / 2^22, so every tile's weights keep 22 bits whatever its scores' distance from the running max. W + 1/2
        // goes to LDS, [head][key], so that the digits' truncation rounds W to nearest (truncation alone would bias
        // every weight down, and the errors would add up). wsc: ws times the digit's weight, for this lane's column.
        float wsc[NG];
#pragma unroll
        for (int ng = 0; ng < NG; ++ng) {
            float w[KB];
            float wmax = 0.0f;
#pragma unroll
            for (int b = 0; b < KB; ++b) {
                const float p = __expf(sc[ng][b] - m[ng]);  // 0 for masked keys (-inf)
                lsum[ng] += p;
                w[b] = p * vscale[b * 16 + c16];
                wmax = fmaxf(wmax, w[b]);
            }
            wmax = group_reduce<16, OpMax>(wmax);  // the tile's largest weight of head kq + 4 ng
            const float inv = wmax > 0.0f ? 4194304.0f / wmax : 0.0f;
#pragma unroll
            for (int b = 0; b < KB; ++b) ptile[(ng * 4 + kq) * kTile + b * 16 + c16] = fmaf(w[b], inv, 0.5f);
            wsc[ng] = __shfl(wmax, 16 * (c16 >> 2), 64) * (1.0f / 4194304.0f) * dscale;
        }
        wave_sync();

        // Weight digits: column (head (c16 / 4) + 4 ng, digit c16 % 4) over keys 16 kq .. + 15.
        i32x4 wd[NG];
#pragma unroll
        for (int ng = 0; ng < NG; ++ng) {
            const float* pw = ptile + (ng * 4 + (c16 >> 2)) * kTile + kq * 16;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const u32x4 w4 = *reinterpret_cast<const u32x4*>(pw + 4 * i);
                uint32_t w[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    w[e] = static_cast<uint32_t>(static_cast<int>(__uint_as_float(w4[e])) + wbias);
                wd[ng][i] = pack_bytes(w[0], w[1], w[2], w[3], dcol);
            }
        }
        // Weighted sum: per 16-dim block, the transposed value codes of keys 16 kq .. + 15 against the digits.
        const int tr_row = kq * 16 + (c16 >> 1);
        const int tr_col = 8 * (c16 & 1);
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const i32x2 lo8 = lds_read_tr8(vt + tr_row * VROW + db * 16 + tr_col);
            const i32x2 hi8 = lds_read_tr8(vt + (tr_row + 8) * VROW + db * 16 + tr_col);
            const i32x4 va = {lo8[0], lo8[1], hi8[0], hi8[1]};
#pragma unroll
            for (int ng = 0; ng < NG; ++ng) {
                const i32x4 zero = {0, 0, 0, 0};
                const i32x4 r4 = __builtin_amdgcn_mfma_i32_16x16x64_i8(va, wd[ng], zero, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) facc[ng][db][r] = fmaf(static_cast<float>(r4[r]), wsc[ng], facc[ng][db][r]);
            }
        }
        wave_sync();  // the tiles are rewritten next time
    }

    // The digit columns of each head add up (lanes 4 g .. 4 g + 3 of each row; the digit-3 column is zero); each
    // head's sum of exponentials is spread over the 16 lanes of its score row.
#pragma unroll
    for (int ng = 0; ng < NG; ++ng) {
        lsum[ng] = group_reduce<16, OpSum>(lsum[ng]);
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
            for (int r = 0; r < 4; ++r) facc[ng][db][r] = group_reduce<4, OpSum>(facc[ng][db][r]);
        }
    }
    // Lane (kq, 4 g') now holds dims 16 db + 4 kq + r of head g' + 4 ng; its max and sum come from row g'.
    const bool writer = (c16 & 3) == 0;
    if (np == 1) {  // uniform: this wave alone covers its head's keys of the split
#pragma unroll
        for (int ng = 0; ng < NG; ++ng) {
            const int g = (c16 >> 2) + 4 * ng;
            const float mg = __shfl(m[ng], 16 * (c16 >> 2), 64);
            const float lg = __shfl(lsum[ng], 16 * (c16 >> 2), 64);
            if (!writer || g >= G) continue;
            const int64_t hh = kvh * G + g;
            if (a.part == nullptr) {
                float* o = a.out + (t * a.q_heads + hh) * D + 4 * kq;
                const float inv = 1.0f / lg;
#pragma unroll
                for (int db = 0; db < DB; ++db)
                    *reinterpret_cast<u32x4*>(o + 16 * db) =
                        u32x4{__float_as_uint(facc[ng][db][0] * inv), __float_as_uint(facc[ng][db][1] * inv),
                              __float_as_uint(facc[ng][db][2] * inv), __float_as_uint(facc[ng][db][3] * inv)};
            } else {
                const int64_t pi = (t * a.q_heads + hh) * a.split + s;  // partial row
                float* pr = a.part + pi * D + 4 * kq;
#pragma unroll
                for (int db = 0; db < DB; ++db)
                    *reinterpret_cast<u32x4*>(pr + 16 * db) =
                        u32x4{__float_as_uint(facc[ng][db][0]), __float_as_uint(facc[ng][db][1]),
                              __float_as_uint(facc[ng][db][2]), __float_as_uint(facc[ng][db][3])};
                if (kq == 0) {
                    float* ml = a.part + a.tokens * a.q_heads * a.split * D + 2 * pi;
                    ml[0] = mg;
                    ml[1] = lg;
                }
            }
        }
        return;
    }
    // Several waves a head: their (max, sum, sums) merge in LDS, over the tiles' space once every wave is done.
    __syncthreads();
    float* const mbuf = reinterpret_cast<float*>(lds);  // [kWaves][G][MROW]
#pragma unroll
    for (int ng = 0; ng < NG; ++ng) {
        const int g = (c16 >> 2) + 4 * ng;
        const float mg = __shfl(m[ng], 16 * (c16 >> 2), 64);
        const float lg = __shfl(lsum[ng], 16 * (c16 >> 2), 64);
        if (!writer || g >= G) continue;
        float* mr = mbuf + (wave * G + g) * MROW;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
            for (int r = 0; r < 4; ++r) mr[16 * db + 4 * kq + r] = facc[ng][db][r];
        }
        if (kq == 0) {
            mr[D] = mg;
            mr[D + 1] = lg;
        }
    }
    __syncthreads();
    // The phase-0 wave of each head merges: lane l takes dims l * D / 64 .. of each of the head's G query heads.
    if (phase != 0) return;
    constexpr int DL = D / 64;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float* m0 = mbuf + (wave * G + g) * MROW;
        float mg = m0[D], lg = m0[D + 1];
        float ag[DL];
#pragma unroll
        for (int i = 0; i < DL; ++i) ag[i] = m0[lane * DL + i];
        for (int p = 1; p < np; ++p) {
            const float* mo = mbuf + ((wave + p * hg) * G + g) * MROW;
            float ao[DL];
#pragma unroll
            for (int i = 0; i < DL; ++i) ao[i] = mo[lane * DL + i];
            merge<DL>(mg, lg, ag, mo[D], mo[D + 1], ao);
        }
        const int64_t hh = kvh * G + g;
        if (a.part == nullptr) {
            float* o = a.out + (t * a.q_heads + hh) * D + lane * DL;
            const float inv = 1.0f / lg;
#pragma unroll
            for (int i = 0; i < DL; ++i) o[i] = ag[i] * inv;
        } else {
            const int64_t pi = (t * a.q_heads + hh) * a.split + s;  // partial row
            float* pr = a.part + pi * D;
#pragma unroll
            for (int i = 0; i < DL; ++i) pr[lane * DL + i] = ag[i];
            if (lane == 0) {
                float* ml = a.part + a.tokens * a.q_heads * a.split * D + 2 * pi;
                ml[0] = mg;
                ml[1] = lg;
            }
        }
    }
}

// out [rows, D] from `split` partial results per row: sums part [rows, split, D], then (max, sum of exponentials)
// pairs ml [rows, split, 2] (the scratch holds the two arrays back to back). A workgroup takes kCombineDims dims of one
// row: thread (split group g, 4-dim group) loads the partial sums of splits g, g + 32, ... (all of them, up to
// kMaxSplit, in one round of loads), and thread s the (max, sum) of split s; so every load is issued before the first
// wait. The maximum, the weights exp(max_s - max) and the denominator come from LDS reductions; the 32 split groups'
// weighted sums add up in LDS.
constexpr int kMaxSplit = 256;
constexpr int kCombineDims = 32;

__global__ __launch_bounds__(256) void attention_combine_rows(const float* part, float* out, int split, int64_t D,
                                                              int64_t rows) {
    constexpr int kD4 = kCombineDims / 4;  // 4-dim groups a workgroup
    constexpr int kGroups = 256 / kD4;     // split groups
    constexpr int kPer = kMaxSplit / kGroups;
    __shared__ float weight[kMaxSplit];
    __shared__ float red[2][4];
    __shared__ u32x4 acc4[kGroups][kD4];
    const uint32_t chunks = static_cast<uint32_t>(D / kCombineDims);
    const int64_t r = blockIdx.x / chunks;
    const int64_t d0 = (blockIdx.x - static_cast<uint32_t>(r) * chunks) * kCombineDims;
    const int tid = threadIdx.x;
    const int d4 = tid % kD4, grp = tid / kD4;
    const float* ml = part + rows * split * D + r * split * 2;
    const float2 mls = *reinterpret_cast<const float2*>(ml + 2 * (tid < split ? tid : split - 1));
    const float ms = tid < split ? mls.x : -INFINITY, ls = tid < split ? mls.y : 0.0f;
    u32x4 v[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int sp = grp + u * kGroups < split ? grp + u * kGroups : split - 1;  // weight 0 past the last split
        v[u] = ld128(part + (r * split + sp) * D + d0 + 4 * d4);
    }
    float mx = group_reduce<64, OpMax>(ms);
    if ((tid & 63) == 0) red[0][tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    const float w = ms == -INFINITY ? 0.0f : __expf(ms - mx);  // splits without keys (max -inf) weigh nothing
    if (tid < kMaxSplit) weight[tid] = w;
    float den = group_reduce<64, OpSum>(ls * w);
    if ((tid & 63) == 0) red[1][tid >> 6] = den;
    __syncthreads();
    den = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int sp = grp + u * kGroups;
        const float ws = sp < split ? weight[sp] : 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] += __uint_as_float(v[u][e]) * ws;
    }
    acc4[grp][d4] = u32x4{__float_as_uint(acc[0]), __float_as_uint(acc[1]), __float_as_uint(acc[2]),
                          __float_as_uint(acc[3])};
    __syncthreads();
    if (tid < kCombineDims) {
        const int dd = tid / 4, e = tid % 4;
        float sum = 0.0f;
#pragma unroll 8
        for (int g = 0; g < kGroups; ++g) sum += __uint_as_float(acc4[g][dd][e]);
        out[r * D + d0 + tid] = sum / den;
    }
}

// ---- Decode attention over float and TurboQuant caches ------------------------------------------------------------
//
// One reader for the pairs of formats the int8 reader above does not take (reference src/backend/sycl/
// sycl_kernels.h:209-212, 236-240; rows as sycl_kv_rows.h's FloatRows, I8Rows and TurboRows):
//  - the Float KV format (SessionOptions::kv Float: f16 rows at f16 precision, f32 at f32; src/quant/kv_format.h:12,
//    sycl_backend.cpp:2224-2228): keys and values [N, Hkv, D] of f16 or f32, sycl_be::attention_rows<KV>;
//  - keys and values in the same TurboQuant format, or int8 keys with TurboQuant values: sycl_be::
//    attention_rows_quantized.
// Semantics: cpu_ref::attention over the values the cache stores (the rows as they are; quant::round_trip_kv: a
// TurboQuant row's decoded values rotated back, an int8 row's fl32(code * scale)). A TurboQuant format keeps its rows
// rotated (each group of 128 values: sign flips, Walsh-Hadamard, 1 / sqrt(128), sign flips), an orthogonal map: the
// query rotated the same way has the originals' dot products with the stored keys, and the weighted sum of stored
// values, rotated back, is the weighted sum of the originals (up to f32 rounding: the reference's device tolerance for
// a quantized cache, tests/unit/backend/device_attention.cpp:23-27).
//
// Layout: one 256-thread workgroup per (token, KV head, key split) for all G query heads, so each key and value row is
// read once for them; the split's keys in tiles of 256, one online softmax per head.
//  - Scores: 8 lanes a key, lane l the LV values LV l .. LV l + LV - 1 of each group of 8 LV values of the row (LV =
//    16, or 8 for head_dim 64; for TurboQuant two of the format's 8-value lanes), 8 keys at once a wave, each lane's
//    loads contiguous. A lane's dot products with the (rotated) query, held in registers where it fits, sum
//    q[d] * x_d over its values (x: the row's value, an int8 code, or a TurboQuant centroid, times the group's norm);
//    int8 keys take the row's scale at the end; 3 DPP steps add the 8 lanes' sums. The scores go through LDS to
//    thread-per-key form for the tile's max and exponentials.
//  - Weighted sum: thread t holds 8 dims of every head (for TurboQuant, the 8 values format lane t % 16 of a group
//    stores) over the tile's keys t / (D / 8) + kS u (kS = 2048 / D key subsets), u = 0, 1, ...: acc += (p * f) * x
//    with f the group's norm (1 for float rows).
//  - TurboQuant codes become centroids through an LDS table indexed by a byte of codes (turbo4: a byte is 2 codes, one
//    64-bit read; turbo2: 4 codes, one 128-bit read; turbo3: 2 low-bit pairs and their 2 third bits, 6 bits, one 64-bit
//    read).
// The value rows a thread adds up are loaded 16 (f32: 8) at a time, the first of them before the scores so that their
// latency overlaps that work. At the end each head's sums add up over the key subsets (and, for TurboQuant values, 16
// threads a group of 128 rotate them back); with one split the workgroup writes the output, with several the partial
// rows with their (max, sum) as the int8 reader writes them.
constexpr int kRowsTile = 256;

// The storage formats, as template arguments: TurboQuant bits 2, 3, 4; 8: int8 codes; 16: f16; 32: f32.
constexpr bool is_turbo(int f) { return f <= 4; }

// Workgroups a CU the rows kernel is compiled for (its four waves a workgroup put as many waves on each SIMD): three
// where the scores run on the matrix cores at head_dim <= 128 with up to 4 query heads a KV head (f16 and int8 keys),
// which then load half as many value rows and key blocks at once to fit 168 registers; two otherwise, as the
// registers fall (TurboQuant and f32 keys need the registers of their lane-wise decode; more heads, their sums). Measured on MI355X at 65,536 keys x 8 KV heads, 32 query heads, head_dim 128, each at its best
// split: f16 rows 58.8 us at three (split 96) against 63.9 at two (split 64); int8 keys with turbo4 values 52.7 against
// 57.6; turbo4 keys at three spill registers and took 64.4 against 50.6.
constexpr int rows_waves(int kf, int d, int g) { return (kf == 16 || kf == 8) && d <= 128 && g <= 4 ? 3 : 2; }
// Bytes of 8 LV values of a row in format f (one group: 128 values for TurboQuant).
constexpr int group_bytes_of(int f, int lv) { return is_turbo(f) ? turbo::group_bytes(f) : 8 * lv * f / 8; }

// The byte-indexed decode table of a TurboQuant format in LDS (entry i: the centroids of the codes byte i holds, as
// above), filled by the workgroup.
template <int Bits>
struct TurboTable {
    static constexpr int kEntries = Bits == 3 ? 64 : 256;
    static constexpr int kWidth = Bits == 2 ? 4 : 2;  // centroids an entry
    __device__ static void fill(float* t, int tid) {
        for (int i = tid; i < kEntries; i += 256) {
            if constexpr (Bits == 4) {
                t[2 * i] = turbo::centroid<4>(i & 15);
                t[2 * i + 1] = turbo::centroid<4>(i >> 4);
            } else if constexpr (Bits == 2) {
#pragma unroll
                for (int e = 0; e < 4; ++e) t[4 * i + e] = turbo::centroid<2>((i >> (2 * e)) & 3);
            } else {
                t[2 * i] = turbo::centroid<3>((i & 3) | (((i >> 4) & 1) << 2));
                t[2 * i + 1] = turbo::centroid<3>(((i >> 2) & 3) | (((i >> 5) & 1) << 2));
            }
        }
    }
    // The 8 centroids of one format lane's codes (turbo::LaneCodes' low and high words).
    __device__ static void decode8(const float* t, uint32_t low, uint32_t high, float* x) {
        if constexpr (Bits == 4) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float2 v = reinterpret_cast<const float2*>(t)[(low >> (8 * i)) & 0xffu];
                x[2 * i] = v.x;
                x[2 * i + 1] = v.y;
            }
        } else if constexpr (Bits == 2) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const float4 v = reinterpret_cast<const float4*>(t)[(low >> (8 * i)) & 0xffu];
                x[4 * i] = v.x;
                x[4 * i + 1] = v.y;
                x[4 * i + 2] = v.z;
                x[4 * i + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t idx = ((low >> (4 * i)) & 15u) | (((high >> (2 * i)) & 3u) << 4);
                const float2 v = reinterpret_cast<const float2*>(t)[idx];
                x[2 * i] = v.x;
                x[2 * i + 1] = v.y;
            }
        }
    }
};

// Widens n 16-bit or 32-bit float values held in raw words.
template <int F>
__device__ __forceinline__ void widen_words(const uint32_t* w, float* x, int n) {
#pragma unroll
    for (int i = 0; i < n; ++i) {
        if constexpr (F == 16) x[i] = f16_to_f32(static_cast<uint16_t>((w[i / 2] >> (16 * (i & 1))) & 0xffffu));
        else x[i] = __uint_as_float(w[i]);
    }
}

// A key lane's LV values of one group, as stored: TurboQuant format lanes 2 l and 2 l + 1 (turbo4: 8 bytes; turbo2:
// 4 bytes; turbo3: those 4 low-bit bytes and 2 third-bit bytes); int8: LV codes; f16 / f32: LV values.
template <int F, int LV>
struct KeyLane {
    static constexpr int kWords = is_turbo(F) ? 2 : LV * F / 32;
    uint32_t w[kWords];
    __device__ __forceinline__ void load(const uint8_t* gc, int l8) {
        if constexpr (F == 4) {
            const uint2 v = *reinterpret_cast<const uint2*>(gc + 8 * l8);
            w[0] = v.x;
            w[1] = v.y;
        } else if constexpr (F == 3 || F == 2) {
            w[0] = *reinterpret_cast<const uint32_t*>(gc + 4 * l8);
            w[1] = F == 3 ? *reinterpret_cast<const uint16_t*>(gc + turbo::kGroup / 4 + 2 * l8) : 0u;
        } else if constexpr (kWords == 2) {
            const uint2 v = *reinterpret_cast<const uint2*>(gc + 8 * l8);
            w[0] = v.x;
            w[1] = v.y;
        } else {
#pragma unroll
            for (int i = 0; i < kWords / 4; ++i) {
                const u32x4 v = ld128_nt(gc + 4 * kWords * l8 + 16 * i);
#pragma unroll
                for (int j = 0; j < 4; ++j) w[4 * i + j] = v[j];
            }
        }
    }
    // The lane's LV values (centroids, int8 codes as floats, or the floats).
    __device__ __forceinline__ void decode(const float* t, float* x) const {
        if constexpr (F == 8) {
#pragma unroll
            for (int b = 0; b < LV; ++b) x[b] = byte_f32(w[b / 4], b % 4);
        } else if constexpr (F == 16 || F == 32) {
            widen_words<F>(w, x, LV);
        } else if constexpr (F == 4) {
            TurboTable<4>::decode8(t, w[0], 0, x);
            TurboTable<4>::decode8(t, w[1], 0, x + 8);
        } else if constexpr (F == 2) {
            TurboTable<2>::decode8(t, w[0] & 0xffffu, 0, x);
            TurboTable<2>::decode8(t, w[0] >> 16, 0, x + 8);
        } else {
            TurboTable<3>::decode8(t, w[0] & 0xffffu, w[1] & 0xffu, x);
            TurboTable<3>::decode8(t, w[0] >> 16, w[1] >> 8, x + 8);
        }
    }
};

// A value thread's 8 dims of one row, as stored: a TurboQuant format lane's codes and the group's f16 norm, or 8 f16 /
// f32 values.
template <int F>
struct ValueSlice {
    static constexpr int kWords = is_turbo(F) ? 2 : F / 4;
    uint32_t w[kWords];
    uint32_t norm = 0;
    // gc: the row's group of this thread's dims; vlane: their slice of it; nb: the group's norm.
    __device__ __forceinline__ void load(const uint8_t* gc, int vlane, const uint16_t* nb) {
        if constexpr (is_turbo(F)) {
            turbo::LaneCodes<F> lc;
            lc.load(gc, vlane);
            w[0] = lc.low;
            w[1] = lc.high;
            norm = *nb;
        } else {
#pragma unroll
            for (int i = 0; i < kWords / 4; ++i) {
                const u32x4 v = ld128_nt(gc + 4 * kWords * vlane + 16 * i);
#pragma unroll
                for (int j = 0; j < 4; ++j) w[4 * i + j] = v[j];
            }
        }
    }
    // The 8 values, to be multiplied by factor().
    __device__ __forceinline__ void decode(const float* t, float* x) const {
        if constexpr (is_turbo(F)) TurboTable<F>::decode8(t, w[0], w[1], x);
        else widen_words<F>(w, x, 8);
    }
    __device__ __forceinline__ float factor() const {
        if constexpr (is_turbo(F)) return f16_to_f32(static_cast<uint16_t>(norm));
        else return 1.0f;
    }
};

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// The scale of the TurboQuant centroids in the f16 key table: 64 c stays a normal f16 in its low part too.
constexpr float kKeyTableScale = 64.0f;

// The key table of a TurboQuant format for the matrix cores: entry i (indexed as TurboTable) holds the f16 high and
// low parts of 64 x the centroids byte i holds -- hi = f16(64 c), lo = f16(64 c - hi), 22 significant bits -- as packed
// pairs: turbo4 / turbo3 {hi pair, lo pair}; turbo2 {hi pair 0, hi pair 1, lo pair 0, lo pair 1}.
template <int Bits>
struct TurboKeyTable {
    static constexpr int kEntries = TurboTable<Bits>::kEntries;
    static constexpr int kWords = Bits == 2 ? 4 : 2;
    __device__ static uint32_t pair(float a, float b) {
        const _Float16 ha = static_cast<_Float16>(a), hb = static_cast<_Float16>(b);
        return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, ha)) |
               (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, hb)) << 16);
    }
    __device__ static void fill(uint32_t* t, int tid) {
        for (int i = tid; i < kEntries; i += 256) {
            float c[4];
            if constexpr (Bits == 4) {
                c[0] = turbo::centroid<4>(i & 15);
                c[1] = turbo::centroid<4>(i >> 4);
            } else if constexpr (Bits == 2) {
#pragma unroll
                for (int e = 0; e < 4; ++e) c[e] = turbo::centroid<2>((i >> (2 * e)) & 3);
            } else {
                c[0] = turbo::centroid<3>((i & 3) | (((i >> 4) & 1) << 2));
                c[1] = turbo::centroid<3>(((i >> 2) & 3) | (((i >> 5) & 1) << 2));
            }
            constexpr int kN = Bits == 2 ? 4 : 2;
            float hi[4], lo[4];
#pragma unroll
            for (int e = 0; e < kN; ++e) {
                const float v = c[e] * kKeyTableScale;
                hi[e] = static_cast<float>(static_cast<_Float16>(v));
                lo[e] = v - hi[e];
            }
            if constexpr (Bits == 2) {
                t[4 * i] = pair(hi[0], hi[1]);
                t[4 * i + 1] = pair(hi[2], hi[3]);
                t[4 * i + 2] = pair(lo[0], lo[1]);
                t[4 * i + 3] = pair(lo[2], lo[3]);
            } else {
                t[2 * i] = pair(hi[0], hi[1]);
                t[2 * i + 1] = pair(lo[0], lo[1]);
            }
        }
    }
    // One format lane's 8 codes (low and high words as turbo::LaneCodes) as the f16 high and low parts of 64 x their
    // centroids, in the matrix-core operand layout (value e in half e).
    __device__ static void decode8(const uint32_t* t, uint32_t low, uint32_t high, uint32_t* hi, uint32_t* lo) {
        if constexpr (Bits == 4) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint2 v = reinterpret_cast<const uint2*>(t)[(low >> (8 * i)) & 0xffu];
                hi[i] = v.x;
                lo[i] = v.y;
            }
        } else if constexpr (Bits == 2) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint4 v = reinterpret_cast<const uint4*>(t)[(low >> (8 * i)) & 0xffu];
                hi[2 * i] = v.x;
                hi[2 * i + 1] = v.y;
                lo[2 * i] = v.z;
                lo[2 * i + 1] = v.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t idx = ((low >> (4 * i)) & 15u) | (((high >> (2 * i)) & 3u) << 4);
                const uint2 v = reinterpret_cast<const uint2*>(t)[idx];
                hi[i] = v.x;
                lo[i] = v.y;
            }
        }
    }
};

__device__ __forceinline__ half8_t as_half8(const uint32_t* w) {
    u32x4 v = {w[0], w[1], w[2], w[3]};
    return __builtin_bit_cast(half8_t, v);
}

// KF, VF: the keys' and the values' formats (both 16 or both 32; or VF TurboQuant with KF the same or 8).
template <int KF, int VF, int G, int D, bool CAP>
__global__ __launch_bounds__(256, rows_waves(KF, D, G) == 3 ? 3 : 1) void attention_rows_kernel(AttnArgs a, const uint8_t* kc, const void* ks,
                                                             const uint8_t* vc, const uint16_t* vn) {
    using namespace turbo;
    static_assert((KF == VF && !is_turbo(KF) && KF != 8) || (is_turbo(VF) && (KF == VF || KF == 8)), "format pair");
    static_assert(!is_turbo(VF) || D % kGroup == 0, "TurboQuant rows are whole groups of 128");
    constexpr int kLV = D == 64 ? 8 : 16;   // values a key lane takes of each group
    constexpr int kGV = 8 * kLV;            // values a group
    constexpr int kNG = D / kGV;            // groups a row
    constexpr int kD8 = D / kLaneValues;    // 8-dim slices a row
    constexpr int kS = 256 / kD8;           // key subsets of the weighted sum
    constexpr int kRowsPerThread = kRowsTile / kS;  // value rows a thread adds up a tile (8 to 64)
    // Of them, loaded together: about 32 words of registers (16 at three waves a SIMD).
    constexpr int kVW = rows_waves(KF, D, G) == 3 ? 16 : 32;
    constexpr int kVB = kVW / ValueSlice<VF>::kWords < 16 ? kVW / ValueSlice<VF>::kWords : 16;
    constexpr int kVPref = kVB < kRowsPerThread ? kVB : kRowsPerThread;
    constexpr int kSets = 256 / 8;          // 8-lane sets that score keys
    constexpr int kKeysPerSet = kRowsTile / kSets;
    // Keys a set loads at once: about 32 words of registers.
    constexpr int kKW = kNG * KeyLane<KF, kLV>::kWords;
    constexpr int kKB = kKW >= 32 ? 1 : 32 / kKW < 8 ? 32 / kKW : 8;
    // Scores on the matrix cores (v_mfma_f32_16x16x32_f16) for f16 and int8 keys up to head_dim 256; f32 and TurboQuant
    // keys, and head_dim 512, take the lanes' fused multiply-adds (measured on MI355X: TurboQuant keys decoded into
    // the matrix operands' f16 high and low parts ran slower than the lanes' decode and multiply-adds).
    constexpr bool kMfma = (KF == 16 || KF == 8) && D <= 256;
    constexpr bool kQReg = !kMfma && G * kNG * kLV <= 64;  // the query values a key lane needs, in registers
    constexpr int kSteps = D / 32;  // 32-dim steps of a key row
    constexpr int kAW = KF == 16 ? 4 : KF == 8 ? 2 : KF == 3 ? 2 : 1;  // words of a lane's A operand a step, as stored
    constexpr int kABlk = kSteps * kAW * 4 <= 64 && rows_waves(KF, D, G) == 2 ? 4 : 2;  // 16-key blocks loaded together
    constexpr int kKGB = group_bytes_of(KF, kLV);
    constexpr int kVGB = group_bytes_of(VF, kLV);
    constexpr int kTab = is_turbo(VF) ? TurboTable<(is_turbo(VF) ? VF : 4)>::kEntries *
                                            TurboTable<(is_turbo(VF) ? VF : 4)>::kWidth
                                      : 1;
    __shared__ __align__(16) float q_s[G][D];
    __shared__ float p_s[G][kRowsTile];
    __shared__ float s_s[G][kRowsTile];
    __shared__ float red[2][4][G];
    __shared__ __align__(16) float acc_s[kS][D];
    __shared__ __align__(16) float tab[kTab];
    __shared__ __align__(16) uint32_t ktab[kMfma && is_turbo(KF) ? TurboKeyTable<(is_turbo(KF) ? KF : 4)>::kEntries *
                                                                        TurboKeyTable<(is_turbo(KF) ? KF : 4)>::kWords
                                                                  : 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t t = blockIdx.y / a.kv_heads;
    const int64_t kvh = blockIdx.y - t * a.kv_heads;
    const int sp = blockIdx.x;

    if constexpr (is_turbo(VF)) TurboTable<VF>::fill(tab, tid);
    if constexpr (kMfma && is_turbo(KF)) TurboKeyTable<KF>::fill(ktab, tid);
    for (int i = tid; i < G * D; i += 256) q_s[i / D][i % D] = a.q[(t * a.q_heads + kvh * G + i / D) * D + i % D];
    if constexpr (is_turbo(KF)) {
        // The query into the keys' rotated domain: 16 threads a group of 128, 8 values each (G * D / 8 is a multiple
        // of 16, so whole groups of 16 lanes take part).
        __syncthreads();
        for (int i = tid; i < G * kD8; i += 256) {
            float* qv = &q_s[i / kD8][(i % kD8) * kLaneValues];
            float v[kLaneValues];
#pragma unroll
            for (int e = 0; e < kLaneValues; ++e) v[e] = qv[e];
            rotate8(v, i % kLanes, false);
#pragma unroll
            for (int e = 0; e < kLaneValues; ++e) qv[e] = v[e];
        }
    }

    int64_t first, last;
    key_range(a, keys_of(a), t, first, last);
    const int64_t len = last >= first ? last - first + 1 : 0;
    const int64_t per = (len + a.split - 1) / a.split;
    const int64_t k0 = first + sp * per;
    const int64_t k1 = k0 + per - 1 < last ? k0 + per - 1 : last;
    float m[G], l[G], acc[G][kLaneValues];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.0f;
#pragma unroll
        for (int e = 0; e < kLaneValues; ++e) acc[g][e] = 0.0f;
    }
    const int dg = tid % kD8, sub = tid / kD8;
    // The group of this thread's 8 value dims and their slice of it (for TurboQuant, the format lane).
    const int vgi = dg / (kGV / kLaneValues), vlane = dg % (kGV / kLaneValues);
    const int set = tid / 8, l8 = tid % 8;  // the 8-lane set and lane that score keys
    __syncthreads();
    float qreg[kQReg ? G : 1][kQReg ? kNG : 1][kLV];
    if constexpr (kQReg) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int gi = 0; gi < kNG; ++gi)
#pragma unroll
                for (int e = 0; e < kLV; ++e) qreg[g][gi][e] = q_s[g][gi * kGV + kLV * l8 + e];
    }
    const uint16_t* knorm = static_cast<const uint16_t*>(ks);
    // The matrix cores' B operand: column n = lane % 16 is query head n (zero past G), rows 8 (lane / 16) + e of each
    // 32-dim step; the query times a power of two qs that brings max |q| just under 2^14, as f16 high and low parts
    // (22 significant bits; qs is undone, exactly, on the scores).
    uint32_t qb_hi[kMfma ? kSteps : 1][4], qb_lo[kMfma ? kSteps : 1][4];
    float q_unscale = 1.0f;
    if constexpr (kMfma) {
        float amax = 0.0f;
        for (int i = tid; i < G * D; i += 256) amax = fmaxf(amax, fabsf(q_s[i / D][i % D]));
        amax = wave_reduce<OpMax>(amax, 0.0f);
        if (lane == 0) red[0][wave][0] = amax;
        __syncthreads();
        amax = fmaxf(fmaxf(red[0][0][0], red[0][1][0]), fmaxf(red[0][2][0], red[0][3][0]));
        int e2 = 0;
        frexpf(amax, &e2);  // amax < 2^e2
        const float qs = amax > 0.0f && amax <= 3.0e38f ? ldexpf(1.0f, 14 - e2) : 1.0f;
        q_unscale = 1.0f / qs;  // a power of two: exact
        const int hn = lane % 16, kq = 8 * (lane / 16);
#pragma unroll
        for (int st = 0; st < kSteps; ++st) {
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                float h[2], lo2[2];
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const float v = hn < G ? q_s[hn < G ? hn : 0][32 * st + kq + e + j] * qs : 0.0f;
                    h[j] = static_cast<float>(static_cast<_Float16>(v));
                    lo2[j] = v - h[j];
                }
                qb_hi[st][e / 2] = TurboKeyTable<4>::pair(h[0], h[1]);
                qb_lo[st][e / 2] = TurboKeyTable<4>::pair(lo2[0], lo2[1]);
            }
        }
        __syncthreads();  // red is rewritten by the first tile
    }
    for (int64_t j0 = k0; j0 <= k1; j0 += kRowsTile) {
        const int64_t n = k1 - j0 + 1 < kRowsTile ? k1 - j0 + 1 : kRowsTile;
        // The value rows this thread adds up in this tile are keys sub + kS u; the first kVPref are requested before
        // the scores.
        ValueSlice<VF> vs[kVPref];
        const auto load_values = [&](int u0) {
#pragma unroll
            for (int u = 0; u < kVPref; ++u) {
                const int k = sub + (u0 + u) * kS;
                const int64_t group = ((j0 + (k < n ? k : 0)) * a.kv_heads + kvh) * kNG + vgi;
                vs[u].load(vc + group * kVGB, vlane, vn + group);
            }
        };
        load_values(0);
        if constexpr (kMfma) {
            // Scores on the matrix cores: wave w takes keys 64 w .. 64 w + 63 of the tile, 16 a block; lane l loads
            // the A operand of key 16 b + l % 16 (8 values of each 32-dim step from 8 (l / 16)) and receives the
            // scores of keys 16 b + 4 (l / 16) + i for query head l % 16.
            const int kq = 8 * (lane / 16);
#pragma unroll 1
            for (int b0 = 0; b0 < 4; b0 += kABlk) {
                uint32_t araw[kABlk][kSteps][kAW];
#pragma unroll
                for (int bb = 0; bb < kABlk; ++bb) {
                    const int kr = 64 * wave + 16 * (b0 + bb) + lane % 16;
                    const int64_t row = (j0 + (kr < n ? kr : 0)) * a.kv_heads + kvh;
#pragma unroll
                    for (int st = 0; st < kSteps; ++st) {
                        if constexpr (KF == 16) {
                            const u32x4 v = ld128_nt(kc + 2 * (row * D + 32 * st + kq));
#pragma unroll
                            for (int i = 0; i < 4; ++i) araw[bb][st][i] = v[i];
                        } else if constexpr (KF == 8) {
                            const uint2 v = *reinterpret_cast<const uint2*>(kc + row * D + 32 * st + kq);
                            araw[bb][st][0] = v.x;
                            araw[bb][st][1] = v.y;
                        } else {
                            const int gi = st / 4, fl = 4 * (st % 4) + lane / 16;  // group, format lane
                            LaneCodes<KF> lc;
                            lc.load(kc + (row * kNG + gi) * group_bytes(KF), fl);
                            araw[bb][st][0] = lc.low;
                            if constexpr (KF == 3) araw[bb][st][1] = lc.high;
                        }
                    }
                }
#pragma unroll
                for (int bb = 0; bb < kABlk; ++bb) {
                    constexpr int kAcc = is_turbo(KF) ? kNG : 1;  // TurboQuant: one accumulator a group (its norm)
                    f32x4_t cacc[kAcc];
#pragma unroll
                    for (int gi = 0; gi < kAcc; ++gi) cacc[gi] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int st = 0; st < kSteps; ++st) {
                        const int gi = is_turbo(KF) ? st / 4 : 0;
                        const half8_t bh = as_half8(qb_hi[st]), bl = as_half8(qb_lo[st]);
                        if constexpr (KF == 16) {
                            const half8_t ah = as_half8(araw[bb][st]);
                            cacc[gi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, cacc[gi], 0, 0, 0);
                            cacc[gi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, cacc[gi], 0, 0, 0);
                        } else if constexpr (KF == 8) {
                            uint32_t w[4];
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                const uint32_t src = araw[bb][st][i / 2];
                                const int s0 = 16 * (i % 2);
                                w[i] = TurboKeyTable<4>::pair(
                                    static_cast<float>(static_cast<int8_t>((src >> s0) & 0xffu)),
                                    static_cast<float>(static_cast<int8_t>((src >> (s0 + 8)) & 0xffu)));
                            }
                            const half8_t ah = as_half8(w);  // the codes, exact in f16
                            cacc[gi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, cacc[gi], 0, 0, 0);
                            cacc[gi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, cacc[gi], 0, 0, 0);
                        } else {
                            uint32_t hi[4], lo[4];
                            TurboKeyTable<KF>::decode8(ktab, araw[bb][st][0], KF == 3 ? araw[bb][st][kAW - 1] : 0u,
                                                       hi, lo);
                            const half8_t ah = as_half8(hi), al = as_half8(lo);
                            cacc[gi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, cacc[gi], 0, 0, 0);
                            cacc[gi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, cacc[gi], 0, 0, 0);
                            cacc[gi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh, cacc[gi], 0, 0, 0);
                        }
                    }
                    const int hn = lane % 16;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int kk = 64 * wave + 16 * (b0 + bb) + 4 * (lane / 16) + i;
                        const int64_t row = (j0 + (kk < n ? kk : 0)) * a.kv_heads + kvh;
                        float x;
                        if constexpr (is_turbo(KF)) {
                            x = 0.0f;
#pragma unroll
                            for (int gi = 0; gi < kAcc; ++gi) x = fmaf(cacc[gi][i], f16_to_f32(knorm[row * kNG + gi]), x);
                            x *= q_unscale * (1.0f / kKeyTableScale);
                        } else if constexpr (KF == 8) {
                            x = cacc[0][i] * q_unscale * static_cast<const float*>(ks)[row];
                        } else {
                            x = cacc[0][i] * q_unscale;
                        }
                        x *= a.scale;
                        if constexpr (CAP) x = a.softcap * tanhf(x / a.softcap);
                        if (hn < G) s_s[hn < G ? hn : 0][kk] = kk < n ? x : -INFINITY;
                    }
                }
            }
        } else {
        // Scores of keys set + 32 u (u < 8), kKB at a time.
#pragma unroll 1
        for (int ub = 0; ub < kKeysPerSet; ub += kKB) {
            KeyLane<KF, kLV> kl[kKB][kNG];
            float kf[kKB][kNG];
#pragma unroll
            for (int u = 0; u < kKB; ++u) {
                const int kk = set + kSets * (ub + u);
                const int64_t row = (j0 + (kk < n ? kk : 0)) * a.kv_heads + kvh;
#pragma unroll
                for (int gi = 0; gi < kNG; ++gi) {
                    kl[u][gi].load(kc + (row * kNG + gi) * kKGB, l8);
                    if constexpr (is_turbo(KF)) kf[u][gi] = f16_to_f32(knorm[row * kNG + gi]);
                }
                if constexpr (KF == 8) kf[u][0] = static_cast<const float*>(ks)[row];
            }
#pragma unroll
            for (int u = 0; u < kKB; ++u) {
                float dot[G];
#pragma unroll
                for (int g = 0; g < G; ++g) dot[g] = 0.0f;
#pragma unroll
                for (int gi = 0; gi < kNG; ++gi) {
                    float x[kLV];
                    kl[u][gi].decode(tab, x);
#pragma unroll
                    for (int g = 0; g < G; ++g) {
                        float part = 0.0f;
                        if constexpr (kQReg) {
#pragma unroll
                            for (int e = 0; e < kLV; ++e) part = fmaf(qreg[g][gi][e], x[e], part);
                        } else {
                            const float* qg = &q_s[g][gi * kGV + kLV * l8];
#pragma unroll
                            for (int e = 0; e < kLV; e += 4) {
                                const float4 q4 = *reinterpret_cast<const float4*>(qg + e);
                                part = fmaf(q4.x, x[e], part);
                                part = fmaf(q4.y, x[e + 1], part);
                                part = fmaf(q4.z, x[e + 2], part);
                                part = fmaf(q4.w, x[e + 3], part);
                            }
                        }
                        if constexpr (is_turbo(KF)) dot[g] = fmaf(part, kf[u][gi], dot[g]);
                        else dot[g] += part;
                    }
                }
                const int kk = set + kSets * (ub + u);
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    float x = group_reduce<8, OpSum>(dot[g]);
                    if constexpr (KF == 8) x *= kf[u][0];
                    x *= a.scale;
                    if constexpr (CAP) x = a.softcap * tanhf(x / a.softcap);
                    if (l8 == 0) s_s[g][kk] = kk < n ? x : -INFINITY;
                }
            }
        }
        }
        __syncthreads();
        float s[G];
#pragma unroll
        for (int g = 0; g < G; ++g) s[g] = s_s[g][tid];
        // The tile's max per head, then exponentials and their sum.
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float w = wave_reduce<OpMax>(s[g], -INFINITY);
            if (lane == 0) red[0][wave][g] = w;
        }
        __syncthreads();
        float c[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float mt = fmaxf(fmaxf(red[0][0][g], red[0][1][g]), fmaxf(red[0][2][g], red[0][3][g]));
            const float mn = fmaxf(m[g], mt);
            c[g] = m[g] == -INFINITY ? 0.0f : __expf(m[g] - mn);
            m[g] = mn;
            const float p = s[g] == -INFINITY ? 0.0f : __expf(s[g] - mn);
            p_s[g][tid] = p;
            const float w = wave_reduce<OpSum>(p, 0.0f);
            if (lane == 0) red[1][wave][g] = w;
        }
        __syncthreads();
        // The weighted sum of the tile's stored value rows.
#pragma unroll
        for (int g = 0; g < G; ++g) {
            l[g] = l[g] * c[g] + ((red[1][0][g] + red[1][1][g]) + (red[1][2][g] + red[1][3][g]));
#pragma unroll
            for (int e = 0; e < kLaneValues; ++e) acc[g][e] *= c[g];
        }
#pragma unroll 1
        for (int u0 = 0; u0 < kRowsPerThread; u0 += kVPref) {
            if (u0 > 0) {
                if (sub + u0 * kS >= n) break;
                load_values(u0);
            }
#pragma unroll
            for (int u = 0; u < kVPref; ++u) {
                const int k = sub + (u0 + u) * kS;
                if (k >= n) break;
                float x[kLaneValues];
                vs[u].decode(tab, x);
                const float f = vs[u].factor();
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float pf = is_turbo(VF) ? p_s[g][k] * f : p_s[g][k];
#pragma unroll
                    for (int e = 0; e < kLaneValues; ++e) acc[g][e] = fmaf(pf, x[e], acc[g][e]);
                }
            }
        }
        __syncthreads();  // s_s, p_s and red are rewritten by the next tile
    }
    // Per head: the key subsets' sums add up (TurboQuant values: 16 threads a group rotate them back), then the output
    // or the partial row with its (max, sum).
#pragma unroll
    for (int g = 0; g < G; ++g) {
        *reinterpret_cast<u32x4*>(&acc_s[sub][kLaneValues * dg]) =
            u32x4{__float_as_uint(acc[g][0]), __float_as_uint(acc[g][1]), __float_as_uint(acc[g][2]),
                  __float_as_uint(acc[g][3])};
        *reinterpret_cast<u32x4*>(&acc_s[sub][kLaneValues * dg + 4]) =
            u32x4{__float_as_uint(acc[g][4]), __float_as_uint(acc[g][5]), __float_as_uint(acc[g][6]),
                  __float_as_uint(acc[g][7])};
        __syncthreads();
        if (tid < kD8) {  // for TurboQuant kD8 is a multiple of 16: whole groups of 16 lanes
            float v[kLaneValues];
#pragma unroll
            for (int e = 0; e < kLaneValues; ++e) {
                float sum = 0.0f;
#pragma unroll
                for (int q = 0; q < kS; ++q) sum += acc_s[q][kLaneValues * tid + e];
                v[e] = sum;
            }
            if constexpr (is_turbo(VF)) rotate8(v, tid % kLanes, true);
            const int64_t hh = kvh * G + g;
            if (a.part == nullptr) {
                float* o = a.out + (t * a.q_heads + hh) * D + kLaneValues * tid;
#pragma unroll
                for (int e = 0; e < kLaneValues; ++e) o[e] = v[e] / l[g];
            } else {
                const int64_t pi = (t * a.q_heads + hh) * a.split + sp;
                float* o = a.part + pi * D + kLaneValues * tid;
#pragma unroll
                for (int e = 0; e < kLaneValues; ++e) o[e] = v[e];
                if (tid == 0) {
                    float* ml = a.part + a.tokens * a.q_heads * a.split * D + 2 * pi;
                    ml[0] = m[g];
                    ml[1] = l[g];
                }
            }
        }
        __syncthreads();  // acc_s is rewritten for the next head
    }
}

template <int KF, int VF, int G>
int launch_kv_rows_g(hipStream_t s, const AttnArgs& a, const void* k, const void* ks, const void* v,
                  const uint16_t* vn, const char* what) {
    const dim3 grid(static_cast<unsigned>(a.split), static_cast<unsigned>(a.tokens * a.kv_heads));
    const bool cap = a.softcap > 0.0f;
    const auto* kc = static_cast<const uint8_t*>(k);
    const auto* vc = static_cast<const uint8_t*>(v);
#define XS_ROWS_CASE(DIM)                                                                                             \
    case DIM:                                                                                                         \
        if (cap) attention_rows_kernel<KF, VF, G, DIM, true><<<grid, 256, 0, s>>>(a, kc, ks, vc, vn);                 \
        else attention_rows_kernel<KF, VF, G, DIM, false><<<grid, 256, 0, s>>>(a, kc, ks, vc, vn);                    \
        break;
    if constexpr (is_turbo(VF)) {
        switch (a.head_dim) {
            XS_ROWS_CASE(128)
            XS_ROWS_CASE(256)
            XS_ROWS_CASE(512)
            default:
                return fail(XS_HIP_EUNSUPPORTED, std::string(what) + ": head_dim " + std::to_string(a.head_dim) +
                                                     " with TurboQuant values (supported: 128, 256, 512)");
        }
    } else {
        switch (a.head_dim) {
            XS_ROWS_CASE(64)
            XS_ROWS_CASE(128)
            XS_ROWS_CASE(256)
            default:
                return fail(XS_HIP_EUNSUPPORTED, std::string(what) + ": head_dim " + std::to_string(a.head_dim) +
                                                     " (supported: 64, 128, 256)");
        }
    }
#undef XS_ROWS_CASE
    return check_launch(what);
}

template <int KF, int VF>
int launch_kv_rows(hipStream_t s, const AttnArgs& a, const void* k, const void* ks, const void* v, const uint16_t* vn,
                const char* what) {
    switch (a.q_heads / a.kv_heads) {
        case 1: return launch_kv_rows_g<KF, VF, 1>(s, a, k, ks, v, vn, what);
        case 2: return launch_kv_rows_g<KF, VF, 2>(s, a, k, ks, v, vn, what);
        case 3: return launch_kv_rows_g<KF, VF, 3>(s, a, k, ks, v, vn, what);
        case 4: return launch_kv_rows_g<KF, VF, 4>(s, a, k, ks, v, vn, what);
        case 5: return launch_kv_rows_g<KF, VF, 5>(s, a, k, ks, v, vn, what);
        case 6: return launch_kv_rows_g<KF, VF, 6>(s, a, k, ks, v, vn, what);
        case 7: return launch_kv_rows_g<KF, VF, 7>(s, a, k, ks, v, vn, what);
        case 8: return launch_kv_rows_g<KF, VF, 8>(s, a, k, ks, v, vn, what);
        default:
            return fail(XS_HIP_EUNSUPPORTED, std::string(what) + ": " + std::to_string(a.q_heads / a.kv_heads) +
                                                 " query heads per KV head (supported: 1 to 8)");
    }
}

// KV heads a workgroup of `waves` waves: the largest power of two up to `waves` dividing kv_heads.
int heads_per_group(int64_t kv_heads, int waves) {
    int hg = waves;
    while (kv_heads % hg != 0) hg /= 2;
    return hg;
}

template <int G, int D>
void launch_rows(hipStream_t s, AttnArgs a) {
    constexpr int W = waves_for(G, D);
    a.hg = heads_per_group(a.kv_heads, W);
    const dim3 grid(static_cast<unsigned>(a.split), static_cast<unsigned>(a.tokens * (a.kv_heads / a.hg)));
    if (a.softcap > 0.0f) attention_i8_rows<G, D, true><<<grid, 64 * W, 0, s>>>(a);
    else attention_i8_rows<G, D, false><<<grid, 64 * W, 0, s>>>(a);
}

template <int G>
int launch_g(hipStream_t s, const AttnArgs& a) {
    switch (a.head_dim) {
        case 64: launch_rows<G, 64>(s, a); break;
        case 128: launch_rows<G, 128>(s, a); break;
        case 256: launch_rows<G, 256>(s, a); break;
        default:
            return fail(XS_HIP_EUNSUPPORTED, "xs_hip_attention_i8: head_dim " + std::to_string(a.head_dim) +
                                                 " (supported: 64, 128, 256)");
    }
    return check_launch("xs_hip_attention_i8");
}

// The split of the rows kernel's keys that puts per_cu workgroups on each CU, each at least half a tile of keys.
// Measured on MI355X, one query token, 32 query and 8 KV heads, head_dim 128, f16 rows at two workgroups a CU: 65536
// keys 54 us at split 64 (68 at 256, 64 at 32), 16384 keys 23 us at 64, 4096 keys 14 us at 32, 1024 keys 14 us at 8
// or 16. A split that is not a whole number of rounds of the CUs leaves a partial round (f16 rows at three a CU: split
// 96, 58.8 us; 80, 63.9; 112, 78.6).
int64_t rows_split(int per_cu, int64_t tokens, int64_t kv_heads, int64_t kv_len) {
    if (tokens <= 0 || kv_heads <= 0 || kv_len <= 0) return 1;
    const int64_t units = tokens * kv_heads;
    int64_t split = (per_cu * static_cast<int64_t>(device_cus()) + units - 1) / units;
    const int64_t by_len = (kv_len + kRowsTile / 2 - 1) / (kRowsTile / 2);
    if (split > by_len) split = by_len;
    if (split > kMaxSplit) split = kMaxSplit;
    return split < 1 ? 1 : split;
}

}  // namespace
}  // namespace xs_hip

using namespace xs_hip;

extern "C" {

int64_t xs_hip_attention_i8_split(int64_t tokens, int64_t kv_heads, int64_t kv_len) {
    if (tokens <= 0 || kv_heads <= 0 || kv_len <= 0) return 1;
    // Up to a workgroup for every CU, and as many as one tile of keys each: a split's workgroups all take their first
    // tile at once, and a decode step waits on the slowest. A cache of at most two tiles a wave stays in one
    // workgroup, where the combine launch would cost more than the split saves. Measured on MI355X, one query token,
    // head_dim 128: with 16 query and 4 KV heads, 1024 keys 10.2 us (4 splits, two tiles a wave: 13.0), 4096 keys
    // 10.8 us (16 splits: 14.3), 256 keys 9.9 us unsplit or split alike, 128 keys 8.0 us unsplit (9.8 split); with 32
    // and 8, 256 keys 9.9 us split in four (12.9 unsplit), 4096 keys 11.5 us (32 splits: 13.4).
    const int hg = heads_per_group(kv_heads, kMaxWaves);
    const int64_t groups = tokens * (kv_heads / hg);
    int64_t split = (static_cast<int64_t>(device_cus()) + groups - 1) / groups;
    const int64_t by_len = kv_len <= 2 * kTile * (kMaxWaves / hg) ? 1 : kv_len / kTile;
    if (split > by_len) split = by_len;
    if (split > kMaxSplit) split = kMaxSplit;
    return split < 1 ? 1 : split;
}

int64_t xs_hip_attention_rows_split(int64_t tokens, int64_t kv_heads, int64_t kv_len) {
    return rows_split(2, tokens, kv_heads, kv_len);
}

int64_t xs_hip_attention_rows_split_kv(xs_kv_format k_format, xs_dtype kv_dtype, int64_t tokens, int64_t q_heads,
                                       int64_t kv_heads, int64_t kv_len, int64_t head_dim) {
    int kf = 0;
    switch (k_format) {
        case XS_KV_FLOAT: kf = kv_dtype == XS_F16 ? 16 : 32; break;
        case XS_KV_I8: kf = 8; break;
        case XS_KV_TURBO4: kf = 4; break;
        case XS_KV_TURBO3: kf = 3; break;
        case XS_KV_TURBO2: kf = 2; break;
        default: kf = 32; break;
    }
    const int64_t g = kv_heads > 0 && q_heads > 0 ? q_heads / kv_heads : 8;
    return rows_split(rows_waves(kf, static_cast<int>(head_dim < 512 ? head_dim : 512), static_cast<int>(g < 8 ? g : 8)),
                      tokens, kv_heads, kv_len);
}

size_t xs_hip_attention_i8_scratch(int64_t tokens, int64_t q_heads, int64_t head_dim, int64_t split) {
    if (split <= 1 || tokens <= 0 || q_heads <= 0 || head_dim <= 0) return 0;
    return static_cast<size_t>(tokens * q_heads * split * (head_dim + 2)) * sizeof(float);
}

}  // extern "C"

namespace {

// Both entry points: kv_len keys, or (kv_len_dev set) a capacity of kv_len keys of which the kernel reads how many
// the cache holds.
int attention_i8(void* stream, const float* q, const void* k_codes, const void* k_scales, const void* v_codes,
                 const void* v_scales, float* out, int64_t tokens, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                 int64_t kv_len, const int64_t* kv_len_dev, float scale, float softcap, int64_t window, int causal,
                 int64_t split, void* scratch, const char* what) {
    if (tokens < 0 || q_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || kv_len < 0 || window < 0 || split < 1 ||
        q_heads % kv_heads != 0)
        return fail(XS_HIP_EINVAL, std::string(what) + ": q [" + std::to_string(tokens) + ", " +
                                       std::to_string(q_heads) + ", " + std::to_string(head_dim) + "] over " +
                                       std::to_string(kv_len) + " keys of " + std::to_string(kv_heads) +
                                       " KV heads, split " + std::to_string(split));
    if (tokens == 0) return XS_HIP_OK;
    if ((causal || window > 0) && kv_len < tokens)
        return fail(XS_HIP_EINVAL, std::string(what) + ": " + std::to_string(kv_len) + " keys for " +
                                       std::to_string(tokens) + " queries");
    if (kv_len == 0) return fail(XS_HIP_EINVAL, std::string(what) + ": no keys");
    if (q == nullptr || k_codes == nullptr || k_scales == nullptr || v_codes == nullptr || v_scales == nullptr ||
        out == nullptr)
        return fail(XS_HIP_EINVAL, std::string(what) + ": null buffer");
    if (split > 1 && scratch == nullptr)
        return fail(XS_HIP_EINVAL, std::string(what) + ": split " + std::to_string(split) +
                                       " needs xs_hip_attention_i8_scratch bytes of scratch");
    if (split > kMaxSplit || tokens * kv_heads > 65535)
        return fail(XS_HIP_EUNSUPPORTED, std::string(what) + ": launch too large");
    if (kv_heads * head_dim >= (int64_t{1} << 24))
        return fail(XS_HIP_EUNSUPPORTED, std::string(what) + ": key rows of " + std::to_string(kv_heads * head_dim) +
                                             " bytes (at most 2^24 - 1)");
    if (!aligned16(q) || !aligned16(out) || !aligned16(k_codes) || !aligned16(v_codes) || head_dim % 16 != 0 ||
        (split > 1 && reinterpret_cast<uintptr_t>(scratch) % 16 != 0))
        return fail(XS_HIP_EINVAL, std::string(what) + ": q, out, codes and scratch must be 16-byte aligned and "
                                                       "head_dim a multiple of 16");
    AttnArgs a{q, static_cast<const int8_t*>(k_codes), static_cast<const float*>(k_scales),
               static_cast<const int8_t*>(v_codes), static_cast<const float*>(v_scales),
               out, split > 1 ? static_cast<float*>(scratch) : nullptr, tokens, q_heads, kv_heads, head_dim, kv_len,
               window, scale, softcap, causal ? 1 : 0, static_cast<int>(split), 1, kv_len_dev};
    const hipStream_t s = as_stream(stream);
    int rc;
    switch (q_heads / kv_heads) {
        case 1: rc = launch_g<1>(s, a); break;
        case 2: rc = launch_g<2>(s, a); break;
        case 3: rc = launch_g<3>(s, a); break;
        case 4: rc = launch_g<4>(s, a); break;
        case 5: rc = launch_g<5>(s, a); break;
        case 6: rc = launch_g<6>(s, a); break;
        case 7: rc = launch_g<7>(s, a); break;
        case 8: rc = launch_g<8>(s, a); break;
        default:
            return fail(XS_HIP_EUNSUPPORTED, std::string(what) + ": " + std::to_string(q_heads / kv_heads) +
                                                 " query heads per KV head (supported: 1 to 8)");
    }
    if (rc != XS_HIP_OK || split == 1) return rc;
    attention_combine_rows<<<static_cast<unsigned>(tokens * q_heads * (head_dim / kCombineDims)), 256, 0, s>>>(
        static_cast<const float*>(scratch), out, static_cast<int>(split), head_dim, tokens * q_heads);
    return check_launch(what);
}

// ---- The no-allocation entry point ---------------------------------------------------------------------------
//
// Its split partials live in `scratch`, a file-scope device array of kNoAllocScratchBytes that every GPU the library
// runs on holds until the process ends (the loader places it with the code object, zero-filled; nothing needs to
// start at zero: each split writes its partial rows before the combine reads them). In host code the array's name
// stands for a host-side shadow, not a device address: the device address is looked up once per device, with that
// device current, and kept.
constexpr size_t kNoAllocScratchBytes = size_t{8} << 20;
__device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;

// The device address of `scratch` on the current device, or an error code.
int noalloc_scratch(void** out, const char* what) {
    static std::mutex mu;
    static void* addr[kMaxDevices] = {};
    int dev = 0;
    const int rc = check_hip(hipGetDevice(&dev), what);
    if (rc != XS_HIP_OK) return rc;
    if (dev < 0 || dev >= kMaxDevices)
        return fail(XS_HIP_EUNSUPPORTED, std::string(what) + ": device " + std::to_string(dev) + " past " +
                                             std::to_string(kMaxDevices));
    std::lock_guard<std::mutex> lock(mu);
    if (addr[dev] == nullptr) {
        void* p = nullptr;
        const int r = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), what);
        if (r != XS_HIP_OK) return r;
        addr[dev] = p;
    }
    *out = addr[dev];
    return XS_HIP_OK;
}

// Both float entry points: as attention_i8, over rows of kv_dtype (F16 or F32).
int attention_float(void* stream, xs_dtype kv_dtype, const float* q, const void* k, const void* v, float* out,
                    int64_t tokens, int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t kv_len,
                    const int64_t* kv_len_dev, float scale, float softcap, int64_t window, int causal, int64_t split,
                    void* scratch, const char* what) {
    if (tokens < 0 || q_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || kv_len < 0 || window < 0 || split < 1 ||
        q_heads % kv_heads != 0)
        return fail(XS_HIP_EINVAL, std::string(what) + ": q [" + std::to_string(tokens) + ", " +
                                       std::to_string(q_heads) + ", " + std::to_string(head_dim) + "] over " +
                                       std::to_string(kv_len) + " keys of " + std::to_string(kv_heads) +
                                       " KV heads, split " + std::to_string(split));
    if (kv_dtype != XS_F16 && kv_dtype != XS_F32)
        return fail(XS_HIP_EUNSUPPORTED, std::string(what) + ": key and value rows of " + dtype_name(kv_dtype) +
                                             " (supported: f16, f32)");
    if (tokens == 0) return XS_HIP_OK;
    if ((causal || window > 0) && kv_len < tokens)
        return fail(XS_HIP_EINVAL, std::string(what) + ": " + std::to_string(kv_len) + " keys for " +
                                       std::to_string(tokens) + " queries");
    if (kv_len == 0) return fail(XS_HIP_EINVAL, std::string(what) + ": no keys");
    if (q == nullptr || k == nullptr || v == nullptr || out == nullptr)
        return fail(XS_HIP_EINVAL, std::string(what) + ": null buffer");
    if (split > 1 && scratch == nullptr)
        return fail(XS_HIP_EINVAL, std::string(what) + ": split " + std::to_string(split) +
                                       " needs xs_hip_attention_i8_scratch bytes of scratch");
    if (split > kMaxSplit || tokens * kv_heads > 65535)
        return fail(XS_HIP_EUNSUPPORTED, std::string(what) + ": launch too large");
    if (!aligned16(q) || !aligned16(out) || !aligned16(k) || !aligned16(v) || head_dim % 16 != 0 ||
        (split > 1 && reinterpret_cast<uintptr_t>(scratch) % 16 != 0))
        return fail(XS_HIP_EINVAL, std::string(what) + ": q, out, keys, values and scratch must be 16-byte aligned "
                                                       "and head_dim a multiple of 16");
    AttnArgs a{q, nullptr, nullptr, nullptr, nullptr, out, split > 1 ? static_cast<float*>(scratch) : nullptr, tokens,
               q_heads, kv_heads, head_dim, kv_len, window, scale, softcap, causal ? 1 : 0, static_cast<int>(split), 1,
               kv_len_dev};
    const hipStream_t s = as_stream(stream);
    const int rc = kv_dtype == XS_F16 ? launch_kv_rows<16, 16>(s, a, k, nullptr, v, nullptr, what)
                                      : launch_kv_rows<32, 32>(s, a, k, nullptr, v, nullptr, what);
    if (rc != XS_HIP_OK || split == 1) return rc;
    attention_combine_rows<<<static_cast<unsigned>(tokens * q_heads * (head_dim / kCombineDims)), 256, 0, s>>>(
        static_cast<const float*>(scratch), out, static_cast<int>(split), head_dim, tokens * q_heads);
    return check_launch(what);
}

// The format's name as quant::kv_format_name gives it (src/quant/kv_format.cpp:22-31).
const char* kv_format_name(xs_kv_format f) {
    switch (f) {
        case XS_KV_FLOAT: return "auto";
        case XS_KV_I8: return "i8";
        case XS_KV_TURBO4: return "turbo4";
        case XS_KV_TURBO3: return "turbo3";
        case XS_KV_TURBO2: return "turbo2";
    }
    return "?";
}

// Both quantized entry points: the formats' pair checked, int8/int8 to the matrix-core reader, the others to the
// TurboQuant reader.
int attention_quantized(void* stream, xs_kv_format kf, xs_kv_format vf, const float* q, const void* k_codes,
                        const void* k_scales, const void* v_codes, const void* v_scales, float* out, int64_t tokens,
                        int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t kv_len,
                        const int64_t* kv_len_dev, float scale, float softcap, int64_t window, int causal,
                        int64_t split, void* scratch, const char* what) {
    const auto turbo_bits = [](xs_kv_format f) {
        return f == XS_KV_TURBO4 ? 4 : f == XS_KV_TURBO3 ? 3 : f == XS_KV_TURBO2 ? 2 : 0;
    };
    const int kb = kf == XS_KV_I8 ? 8 : turbo_bits(kf), vb = vf == XS_KV_I8 ? 8 : turbo_bits(vf);
    // The pairs kv_formats_supported admits besides float/float: int8/int8, a TurboQuant format for both, int8 keys
    // with TurboQuant values (sycl_kernels.h:209-212).
    if (kb == 0 || vb == 0 || !(kb == vb || (kb == 8 && vb != 8)))
        return fail(XS_HIP_EUNSUPPORTED, std::string(what) + ": keys in " + kv_format_name(kf) + " with values in " +
                                             kv_format_name(vf));
    if (vb == 8)
        return attention_i8(stream, q, k_codes, k_scales, v_codes, v_scales, out, tokens, q_heads, kv_heads, head_dim,
                            kv_len, kv_len_dev, scale, softcap, window, causal, split, scratch, what);
    if (tokens < 0 || q_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || kv_len < 0 || window < 0 || split < 1 ||
        q_heads % kv_heads != 0)
        return fail(XS_HIP_EINVAL, std::string(what) + ": q [" + std::to_string(tokens) + ", " +
                                       std::to_string(q_heads) + ", " + std::to_string(head_dim) + "] over " +
                                       std::to_string(kv_len) + " keys of " + std::to_string(kv_heads) +
                                       " KV heads, split " + std::to_string(split));
    if (head_dim % 128 != 0)
        return fail(XS_HIP_EINVAL, std::string(what) + ": a TurboQuant KV format needs a head_dim that is a multiple "
                                                       "of 128, got " + std::to_string(head_dim));
    if (tokens == 0) return XS_HIP_OK;
    if ((causal || window > 0) && kv_len < tokens)
        return fail(XS_HIP_EINVAL, std::string(what) + ": " + std::to_string(kv_len) + " keys for " +
                                       std::to_string(tokens) + " queries");
    if (kv_len == 0) return fail(XS_HIP_EINVAL, std::string(what) + ": no keys");
    if (q == nullptr || k_codes == nullptr || k_scales == nullptr || v_codes == nullptr || v_scales == nullptr ||
        out == nullptr)
        return fail(XS_HIP_EINVAL, std::string(what) + ": null buffer");
    if (split > 1 && scratch == nullptr)
        return fail(XS_HIP_EINVAL, std::string(what) + ": split " + std::to_string(split) +
                                       " needs xs_hip_attention_i8_scratch bytes of scratch");
    if (split > kMaxSplit || tokens * kv_heads > 65535)
        return fail(XS_HIP_EUNSUPPORTED, std::string(what) + ": launch too large");
    if (!aligned16(q) || !aligned16(out) || !aligned16(k_codes) || !aligned16(v_codes) ||
        reinterpret_cast<uintptr_t>(k_scales) % (kb == 8 ? 4 : 2) != 0 ||
        reinterpret_cast<uintptr_t>(v_scales) % 2 != 0 ||
        (split > 1 && reinterpret_cast<uintptr_t>(scratch) % 16 != 0))
        return fail(XS_HIP_EINVAL, std::string(what) + ": q, out, codes and scratch must be 16-byte aligned, f32 "
                                                       "scales 4-byte and f16 norms 2-byte aligned");
    AttnArgs a{q, nullptr, nullptr, nullptr, nullptr, out, split > 1 ? static_cast<float*>(scratch) : nullptr, tokens,
               q_heads, kv_heads, head_dim, kv_len, window, scale, softcap, causal ? 1 : 0, static_cast<int>(split), 1,
               kv_len_dev};
    const hipStream_t s = as_stream(stream);
    const auto* vn = static_cast<const uint16_t*>(v_scales);
    int rc;
    if (vb == 4) rc = kb == 8 ? launch_kv_rows<8, 4>(s, a, k_codes, k_scales, v_codes, vn, what)
                              : launch_kv_rows<4, 4>(s, a, k_codes, k_scales, v_codes, vn, what);
    else if (vb == 3) rc = kb == 8 ? launch_kv_rows<8, 3>(s, a, k_codes, k_scales, v_codes, vn, what)
                                   : launch_kv_rows<3, 3>(s, a, k_codes, k_scales, v_codes, vn, what);
    else rc = kb == 8 ? launch_kv_rows<8, 2>(s, a, k_codes, k_scales, v_codes, vn, what)
                      : launch_kv_rows<2, 2>(s, a, k_codes, k_scales, v_codes, vn, what);
    if (rc != XS_HIP_OK || split == 1) return rc;
    attention_combine_rows<<<static_cast<unsigned>(tokens * q_heads * (head_dim / kCombineDims)), 256, 0, s>>>(
        static_cast<const float*>(scratch), out, static_cast<int>(split), head_dim, tokens * q_heads);
    return check_launch(what);
}

}  // namespace

extern "C" {

int xs_hip_attention(void* stream, xs_dtype kv_dtype, const float* q, const void* k, const void* v, float* out,
                     int64_t tokens, int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t kv_len, float scale,
                     float softcap, int64_t window, int causal, int64_t split, void* scratch) {
    return attention_float(stream, kv_dtype, q, k, v, out, tokens, q_heads, kv_heads, head_dim, kv_len, nullptr, scale,
                           softcap, window, causal, split, scratch, "xs_hip_attention");
}

int xs_hip_attention_at(void* stream, xs_dtype kv_dtype, const float* q, const void* k, const void* v, float* out,
                        int64_t tokens, int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t kv_capacity,
                        const int64_t* kv_len, float scale, float softcap, int64_t window, int causal, int64_t split,
                        void* scratch) {
    if (kv_len == nullptr || reinterpret_cast<uintptr_t>(kv_len) % 8 != 0)
        return fail(XS_HIP_EINVAL, "xs_hip_attention_at: kv_len must be an 8-byte aligned device int64");
    return attention_float(stream, kv_dtype, q, k, v, out, tokens, q_heads, kv_heads, head_dim, kv_capacity, kv_len,
                           scale, softcap, window, causal, split, scratch, "xs_hip_attention_at");
}

int xs_hip_attention_i8(void* stream, const float* q, const void* k_codes, const void* k_scales, const void* v_codes,
                        const void* v_scales, float* out, int64_t tokens, int64_t q_heads, int64_t kv_heads,
                        int64_t head_dim, int64_t kv_len, float scale, float softcap, int64_t window, int causal,
                        int64_t split, void* scratch) {
    return attention_i8(stream, q, k_codes, k_scales, v_codes, v_scales, out, tokens, q_heads, kv_heads, head_dim,
                        kv_len, nullptr, scale, softcap, window, causal, split, scratch, "xs_hip_attention_i8");
}

int xs_hip_attention_i8_at(void* stream, const float* q, const void* k_codes, const void* k_scales,
                           const void* v_codes, const void* v_scales, float* out, int64_t tokens, int64_t q_heads,
                           int64_t kv_heads, int64_t head_dim, int64_t kv_capacity, const int64_t* kv_len,
                           float scale, float softcap, int64_t window, int causal, int64_t split, void* scratch) {
    if (kv_len == nullptr || reinterpret_cast<uintptr_t>(kv_len) % 8 != 0)
        return fail(XS_HIP_EINVAL, "xs_hip_attention_i8_at: kv_len must be an 8-byte aligned device int64");
    return attention_i8(stream, q, k_codes, k_scales, v_codes, v_scales, out, tokens, q_heads, kv_heads, head_dim,
                        kv_capacity, kv_len, scale, softcap, window, causal, split, scratch, "xs_hip_attention_i8_at");
}

int xs_hip_attention_i8_noalloc(void* stream, const float* q, const void* k_codes, const void* k_scales,
                                const void* v_codes, const void* v_scales, float* out, int64_t tokens, int64_t q_heads,
                                int64_t kv_heads, int64_t head_dim, int64_t kv_len, float scale, float softcap,
                                int64_t window, int causal, int64_t split) {
    const char* what = "xs_hip_attention_i8_noalloc";
    void* buf = nullptr;
    if (split > 1) {
        const size_t need = xs_hip_attention_i8_scratch(tokens, q_heads, head_dim, split);
        if (need > kNoAllocScratchBytes)
            return fail(XS_HIP_EINVAL, std::string(what) + ": split " + std::to_string(split) + " of " +
                                           std::to_string(tokens) + " x " + std::to_string(q_heads) +
                                           " query rows of " + std::to_string(head_dim) + " needs " +
                                           std::to_string(need) + " bytes of scratch; this entry point holds " +
                                           std::to_string(kNoAllocScratchBytes));
        const int rc = noalloc_scratch(&buf, what);
        if (rc != XS_HIP_OK) return rc;
    }
    return attention_i8(stream, q, k_codes, k_scales, v_codes, v_scales, out, tokens, q_heads, kv_heads, head_dim,
                        kv_len, nullptr, scale, softcap, window, causal, split, buf, what);
}

int xs_hip_attention_quantized(void* stream, xs_kv_format k_format, xs_kv_format v_format, const float* q,
                               const void* k_codes, const void* k_scales, const void* v_codes, const void* v_scales,
                               float* out, int64_t tokens, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                               int64_t kv_len, float scale, float softcap, int64_t window, int causal, int64_t split,
                               void* scratch) {
    return attention_quantized(stream, k_format, v_format, q, k_codes, k_scales, v_codes, v_scales, out, tokens,
                               q_heads, kv_heads, head_dim, kv_len, nullptr, scale, softcap, window, causal, split,
                               scratch, "xs_hip_attention_quantized");
}

int xs_hip_attention_quantized_at(void* stream, xs_kv_format k_format, xs_kv_format v_format, const float* q,
                                  const void* k_codes, const void* k_scales, const void* v_codes,
                                  const void* v_scales, float* out, int64_t tokens, int64_t q_heads, int64_t kv_heads,
                                  int64_t head_dim, int64_t kv_capacity, const int64_t* kv_len, float scale,
                                  float softcap, int64_t window, int causal, int64_t split, void* scratch) {
    if (kv_len == nullptr || reinterpret_cast<uintptr_t>(kv_len) % 8 != 0)
        return fail(XS_HIP_EINVAL, "xs_hip_attention_quantized_at: kv_len must be an 8-byte aligned device int64");
    return attention_quantized(stream, k_format, v_format, q, k_codes, k_scales, v_codes, v_scales, out, tokens,
                               q_heads, kv_heads, head_dim, kv_capacity, kv_len, scale, softcap, window, causal, split,
                               scratch, "xs_hip_attention_quantized_at");
}

}  // extern "C"
