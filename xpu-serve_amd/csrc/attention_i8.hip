// Decode attention over an int8 KV cache for gfx950: the reader of the codes and scales xs_hip_quantize_kv writes.
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
// Layout: one workgroup of four waves per (token, KV head, key split); the G query heads sharing the KV head are
// handled together, so each key and value row is read once for all of them. Each wave takes every fourth tile of 64
// consecutive keys of the split: it loads the tile's key codes into LDS and its value codes into registers, whole
// rows per 128-bit load instruction; then a lane per key computes its key's scores against the G heads (q is the same
// for every lane: LDS broadcasts), the tile's max per head moves the wave's running max (rescaling the
// accumulator at most once per tile), and each key's p * v_scale goes to LDS; then each lane accumulates the value
// rows it loaded, 8 dims each, weighted in f32. The lanes sharing dims add up (they share the running max), and the
// four waves' (max, sum, accumulator) merge in LDS at the end. With one split the workgroup writes the output; with
// several it writes [head_dim partial sums, max, sum] rows that a second launch merges (flash decoding).
//
// Accuracy: f32 accumulation where cpu-ref accumulates in f64, and the key scale applied to the dot product rather
// than to each product -- within the reference's own device tolerance for a quantized cache
// (tests/unit/backend/device_attention.cpp:23-27).
#include <cmath>
#include <type_traits>

#include "common.h"

namespace xs_hip {
namespace {

struct AttnArgs {
    const float* q;       // [T, Hq, D]
    const int8_t* kc;     // [N, Hkv, D] key codes
    const float* ks;      // [N, Hkv] key scales
    const int8_t* vc;     // [N, Hkv, D] value codes
    const float* vs;      // [N, Hkv] value scales
    float* out;           // [T, Hq, D], or null when `part` is written
    float* part;          // [T * Hq * split, D + 2], or null
    int64_t tokens, q_heads, kv_heads, head_dim, kv_len, window;
    float scale, softcap;
    int causal, split;
};

// The key range [first, last] of query token t (cpu_ref::attention, ops.cpp:565-575 without blocks and anchors).
__device__ __forceinline__ void key_range(const AttnArgs& a, int64_t t, int64_t& first, int64_t& last) {
    const int64_t pos = a.kv_len - a.tokens + t;
    first = a.window > 0 ? (pos - a.window + 1 > 0 ? pos - a.window + 1 : 0) : 0;
    last = a.causal ? pos : a.kv_len - 1;
    if (a.window > 0 && pos + a.window - 1 < last) last = pos + a.window - 1;
}

constexpr int kWaves = 4;    // waves a workgroup; each takes every fourth tile of 64 keys, and they merge in LDS
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

// q of one head as a 23-bit integer per dim, Q = round(q / qs) with qs = max |q| / 2^22, written as three balanced
// base-256 digits (hi * 65536 + mid * 256 + lo, each in [-128, 127]) so that int8 matrix cores can take it. The
// digits are exact: qs * Q is q within 2^-23 of max |q|.
__device__ __forceinline__ void q_digits(float q, float inv_qs, int& hi, int& mid, int& lo) {
    const int Q = static_cast<int>(rintf(q * inv_qs));
    lo = static_cast<int8_t>(Q & 0xff);
    const int q1 = (Q - lo) >> 8;
    mid = static_cast<int8_t>(q1 & 0xff);
    hi = (q1 - mid) >> 8;
}

typedef int i32x2 __attribute__((ext_vector_type(2)));

// Reads 8 bytes a lane from LDS with the transpose of ds_read_b64_tr_b8: within each group of 16 lanes, with C_j the
// 8 bytes at lane j's address, lane i receives byte i % 8 of C_{2k + i / 8} as its byte k (k < 8). Lane j pointing at
// row base + j / 2, column col + 8 (j % 2) of a row-major byte tile thus gives lane i column col + i of rows
// base .. base + 7: a 16-column by 8-row block, transposed.
__device__ __forceinline__ i32x2 lds_read_tr8(const uint8_t* p) {
    // p points into LDS: the C cast converts the generic address to the LDS address space the builtin takes.
    return __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) i32x2*)(p));
}

// G query heads per KV head, D head_dim (64, 128 or 256).
//
// Both products run on the int8 matrix cores (v_mfma_i32_16x16x64_i8; 16 x 16 results, K = 64):
//  - scores S [16 keys, 16 heads] = key codes [16 keys, 64 dims] x digits of q [64 dims, 16 heads], a 64-dim chunk at
//    a time. Lane l holds 16 codes of key l % 16 (dims 16 (l / 16) ..) -- a plain 16-byte load -- and the digits of
//    head l % 16 over the same dims; it receives the scores of keys 4 (l / 16) + r (r < 4) for head l % 16.
//  - the weighted sum O^T [16 dims, 16 heads] = value codes^T [16 dims, 64 keys] x digits of the weights
//    [64 keys, 16 heads]. The value tile is staged in LDS row-major and read transposed (lds_read_tr8), so lane l
//    holds 16 keys' codes of dim l % 16; the weights w = p * v_scale, as integers W = round(w / ws) with
//    ws = max v_scale / 2^22 over the wave's keys (p <= 1), in three digits. Lane l receives dims 4 (l / 16) + r of
//    head l % 16: exact int32 sums of the tile, added to the f32 accumulator times ws.
template <int G, int D>
__global__ __launch_bounds__(64 * kWaves) void attention_i8_rows(AttnArgs a, const float* __restrict__ qg) {
    constexpr int KC = D / 64;             // 64-dim chunks of a key row: the K of one score step
    constexpr int KB = kTile / 16;         // 16-key blocks of a tile: the M of one score step
    constexpr int DB = D / 16;             // 16-dim blocks of a value row: the M of one weighted-sum step
    constexpr int VROW = D + 8;            // LDS bytes a staged value row (8 bytes of padding: distinct banks for the
                                           // eight rows one transposed read covers)
    constexpr int VLPR = D / 8;            // lanes a value row with 8-byte loads
    constexpr int VRPI = 64 / VLPR;        // value rows one load instruction covers
    constexpr int VI = kTile / VRPI;       // value load instructions a tile
    static_assert(G <= 16, "the query heads of a KV head fill at most the 16 columns of a matrix-core step");
    static_assert(kTile == 64, "a weighted-sum step takes the 64 keys of a tile");
    __shared__ __align__(16) float ptile[kWaves][G][kTile];     // p of each head and key of each wave's tile
    __shared__ __align__(16) float vscale[kWaves][kTile];       // value scales of each wave's tile
    __shared__ __align__(16) float kscale[kWaves][kTile];       // key scales of each wave's tile
    __shared__ __align__(16) uint8_t vtile[kWaves][kTile * VROW];
    __shared__ float mbuf[kWaves][G][D + 2];

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    // Grid (split, token x KV head): consecutive workgroup ids are splits, so the KV heads of one split share an id
    // residue mod 8 -- the same XCD and L2 -- and the lines of key/value rows and scales those heads share are fetched
    // once per XCD rather than once per head.
    const int64_t row = blockIdx.y;  // (t, kv head)
    const int64_t t = row / a.kv_heads;
    const int64_t kvh = row - t * a.kv_heads;
    const int s = blockIdx.x;

    int64_t first, last;
    key_range(a, t, first, last);
    const int64_t len = last >= first ? last - first + 1 : 0;
    const int64_t per = (len + a.split - 1) / a.split;
    const int64_t k0 = first + s * per;
    int64_t k1 = k0 + per - 1;
    if (k1 > last) k1 = last;
    const int64_t span = k1 >= k0 ? k1 - k0 + 1 : 0;
    const int64_t tiles = (span + kTile - 1) / kTile;

    const int h = lane & 15;   // the head (matrix-core column) of this lane
    const int kq = lane >> 4;  // its 16-dim / 16-key / 4-row group

    // q as three digits per dim (the score step's B operand), and its scale.
    i32x4 qd[3][KC];
    float qs_h;
    {
        float qv[KC][16];
        float mx = 0.0f;
        const float* q = qg + (t * a.q_heads + kvh * G + (h < G ? h : 0)) * D;
#pragma unroll
        for (int c = 0; c < KC; ++c) {
#pragma unroll
            for (int i = 0; i < 16; i += 4) {
                const u32x4 raw = ld128(q + c * 64 + kq * 16 + i);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    qv[c][i + e] = h < G ? __uint_as_float(raw[e]) : 0.0f;
                    mx = fmaxf(mx, fabsf(qv[c][i + e]));
                }
            }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));  // max |q| of head h over all its dims
        qs_h = mx / 4194304.0f;
        const float inv = mx > 0.0f ? 4194304.0f / mx : 0.0f;
#pragma unroll
        for (int c = 0; c < KC; ++c) {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                uint32_t dh = 0, dm = 0, dl = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    int hi, mid, lo;
                    q_digits(qv[c][4 * w + e], inv, hi, mid, lo);
                    dh |= static_cast<uint32_t>(hi & 0xff) << (8 * e);
                    dm |= static_cast<uint32_t>(mid & 0xff) << (8 * e);
                    dl |= static_cast<uint32_t>(lo & 0xff) << (8 * e);
                }
                qd[0][c][w] = static_cast<int>(dh);
                qd[1][c][w] = static_cast<int>(dm);
                qd[2][c][w] = static_cast<int>(dl);
            }
        }
    }
    const float score_scale = qs_h * a.scale;

    // The weights' integer scale: the largest value scale among this wave's keys (p <= 1 bounds the weights by it).
    float ws;
    {
        float mv = 0.0f;
        for (int64_t tile = wave; tile < tiles; tile += kWaves) {
            const int64_t j = k0 + tile * kTile + lane;
            if (j <= k1) mv = fmaxf(mv, a.vs[j * a.kv_heads + kvh]);
        }
        mv = group_reduce<64, OpMax>(mv);
        ws = mv / 4194304.0f;
    }
    const float inv_ws = ws > 0.0f ? 1.0f / ws : 0.0f;

    float m[G];                 // the wave's running max per head (the same in every lane)
    float lsum = 0.0f;          // this lane's share of head h's sum of exponentials
    float mh = -INFINITY;       // the running max of head h
    float facc[DB][4];          // head h, dims 16 db + 4 kq + r: the weighted sums
#pragma unroll
    for (int g = 0; g < G; ++g) m[g] = -INFINITY;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
        for (int r = 0; r < 4; ++r) facc[db][r] = 0.0f;
    }

    // The waves run independently: wave w takes tiles w, w + kWaves, ... and touches only its own LDS, whose writes
    // and reads are ordered within the wave (wave_sync).
    auto wave_sync = [] {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    uint8_t* vt = vtile[wave];
    for (int64_t tile = wave; tile < tiles; tile += kWaves) {
        const int64_t j0 = k0 + tile * kTile;  // keys j0 .. j0 + 63 (those past k1 clamped to it, weights 0)
        // Loads: key codes in the score step's A layout, value rows (to LDS), the tile's scales.
        i32x4 kw[KB][KC];
#pragma unroll
        for (int b = 0; b < KB; ++b) {
            int64_t j = j0 + b * 16 + h;
            j = j <= k1 ? j : k1;
            const int8_t* kp = a.kc + (j * a.kv_heads + kvh) * D + kq * 16;
#pragma unroll
            for (int c = 0; c < KC; ++c) kw[b][c] = __builtin_bit_cast(i32x4, ld128_nt(kp + c * 64));
        }
        uint64_t vw[VI];
#pragma unroll
        for (int i = 0; i < VI; ++i) {
            int64_t j = j0 + i * VRPI + lane / VLPR;
            j = j <= k1 ? j : k1;
            vw[i] = __builtin_nontemporal_load(
                reinterpret_cast<const uint64_t*>(a.vc + (j * a.kv_heads + kvh) * D + (lane % VLPR) * 8));
        }
        {
            const int64_t jl = j0 + lane;
            const int64_t rk = (jl <= k1 ? jl : k1) * a.kv_heads + kvh;
            kscale[wave][lane] = a.ks[rk];
            vscale[wave][lane] = a.vs[rk];
        }
#pragma unroll
        for (int i = 0; i < VI; ++i)
            *reinterpret_cast<uint64_t*>(vt + (i * VRPI + lane / VLPR) * VROW + (lane % VLPR) * 8) = vw[i];
        wave_sync();

        // Scores: three digit products per 16-key block and 64-dim chunk, combined in f32.
        float sc[KB][4];
        float mt = -INFINITY;
#pragma unroll
        for (int b = 0; b < KB; ++b) {
            i32x4 r0 = {0, 0, 0, 0}, r1 = {0, 0, 0, 0}, r2 = {0, 0, 0, 0};
#pragma unroll
            for (int c = 0; c < KC; ++c) {
                r0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(kw[b][c], qd[0][c], r0, 0, 0, 0);
                r1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(kw[b][c], qd[1][c], r1, 0, 0, 0);
                r2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(kw[b][c], qd[2][c], r2, 0, 0, 0);
            }
            const u32x4 ks4 = *reinterpret_cast<const u32x4*>(&kscale[wave][b * 16 + kq * 4]);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float dot = static_cast<float>(r0[r]) * 65536.0f + static_cast<float>(r1[r]) * 256.0f +
                                  static_cast<float>(r2[r]);
                float x = dot * score_scale * __uint_as_float(ks4[r]);
                if (a.softcap > 0.0f) x = a.softcap * tanhf(x / a.softcap);
                const bool valid = j0 + b * 16 + kq * 4 + r <= k1;
                sc[b][r] = valid ? x : -INFINITY;
                mt = fmaxf(mt, sc[b][r]);
            }
        }
        mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
        mt = fmaxf(mt, __shfl_xor(mt, 32, 64));  // the tile's max of head h
        // A larger max for some head: flush the digit sums, rescaling each lane's head by exp(old - new).
        const float mn = fmaxf(mh, mt);
        bool moved = false;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float mtg = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mt), g));
            moved |= mtg > m[g];
            m[g] = fmaxf(m[g], mtg);
        }
        if (moved) {  // uniform across the wave
            const float c = mh == -INFINITY ? 0.0f : __expf(mh - mn);
            lsum *= c;
#pragma unroll
            for (int db = 0; db < DB; ++db) {
#pragma unroll
                for (int r = 0; r < 4; ++r) facc[db][r] *= c;
            }
        }
        mh = mn;
        // p = exp(s - max) per (head, key) to LDS; this lane's keys: 16 b + 4 kq + r of head h.
        if (h < G) {
#pragma unroll
            for (int b = 0; b < KB; ++b) {
                float p4[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    p4[r] = __expf(sc[b][r] - mh);  // 0 for keys past the split (-inf)
                    lsum += p4[r];
                }
                *reinterpret_cast<u32x4*>(&ptile[wave][h][b * 16 + kq * 4]) =
                    u32x4{__float_as_uint(p4[0]), __float_as_uint(p4[1]), __float_as_uint(p4[2]),
                          __float_as_uint(p4[3])};
            }
        }
        wave_sync();

        // Weights of head h over keys 16 kq .. + 15, as three digits: the weighted-sum step's B operand.
        i32x4 wd[3];
        {
            float w[16];
#pragma unroll
            for (int i = 0; i < 16; i += 4) {
                const u32x4 p4 = h < G ? *reinterpret_cast<const u32x4*>(&ptile[wave][h][kq * 16 + i]) : u32x4{0, 0, 0, 0};
                const u32x4 v4 = *reinterpret_cast<const u32x4*>(&vscale[wave][kq * 16 + i]);
#pragma unroll
                for (int e = 0; e < 4; ++e) w[i + e] = __uint_as_float(p4[e]) * __uint_as_float(v4[e]);
            }
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                uint32_t dh = 0, dm = 0, dl = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    int hi, mid, lo;
                    q_digits(w[4 * q4 + e], inv_ws, hi, mid, lo);
                    dh |= static_cast<uint32_t>(hi & 0xff) << (8 * e);
                    dm |= static_cast<uint32_t>(mid & 0xff) << (8 * e);
                    dl |= static_cast<uint32_t>(lo & 0xff) << (8 * e);
                }
                wd[0][q4] = static_cast<int>(dh);
                wd[1][q4] = static_cast<int>(dm);
                wd[2][q4] = static_cast<int>(dl);
            }
        }
        // Weighted sum: per 16-dim block, the transposed value codes of keys 16 kq .. + 15 against the digits.
        const int tr_row = kq * 16 + (h >> 1);
        const int tr_col = 8 * (h & 1);
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const i32x2 lo8 = lds_read_tr8(vt + tr_row * VROW + db * 16 + tr_col);
            const i32x2 hi8 = lds_read_tr8(vt + (tr_row + 8) * VROW + db * 16 + tr_col);
            const i32x4 va = {lo8[0], lo8[1], hi8[0], hi8[1]};
            const i32x4 zero = {0, 0, 0, 0};
            const i32x4 r0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(va, wd[0], zero, 0, 0, 0);
            const i32x4 r1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(va, wd[1], zero, 0, 0, 0);
            const i32x4 r2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(va, wd[2], zero, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float v = static_cast<float>(r0[r]) * 65536.0f + static_cast<float>(r1[r]) * 256.0f +
                                static_cast<float>(r2[r]);
                facc[db][r] = fmaf(v, ws, facc[db][r]);
            }
        }
        wave_sync();  // the tiles are rewritten next time
    }

    // Each head's sum of exponentials is spread over the lanes of that head. Then the four waves merge through LDS;
    // lane l holds dims 16 db + 4 kq + r of head h.
    lsum += __shfl_xor(lsum, 16, 64);
    lsum += __shfl_xor(lsum, 32, 64);
    if (h < G) {
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
            for (int r = 0; r < 4; ++r) mbuf[wave][h][db * 16 + kq * 4 + r] = facc[db][r];
        }
        if (kq == 0) {
            mbuf[wave][h][D] = mh;
            mbuf[wave][h][D + 1] = lsum;
        }
    }
    __syncthreads();
    // Wave 0 merges: lane l takes dims l * D / 64 .. of every head.
    if (wave != 0) return;
    constexpr int DL = D / 64;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float mg = mbuf[0][g][D], lg = mbuf[0][g][D + 1];
        float ag[DL];
#pragma unroll
        for (int i = 0; i < DL; ++i) ag[i] = mbuf[0][g][lane * DL + i];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) {
            float ao[DL];
#pragma unroll
            for (int i = 0; i < DL; ++i) ao[i] = mbuf[w][g][lane * DL + i];
            merge<DL>(mg, lg, ag, mbuf[w][g][D], mbuf[w][g][D + 1], ao);
        }
        const int64_t hh = kvh * G + g;
        if (a.part == nullptr) {
            float* o = a.out + (t * a.q_heads + hh) * D + lane * DL;
            const float inv = 1.0f / lg;
#pragma unroll
            for (int i = 0; i < DL; ++i) o[i] = ag[i] * inv;
        } else {
            float* pr = a.part + ((t * a.q_heads + hh) * a.split + s) * (D + 2);
#pragma unroll
            for (int i = 0; i < DL; ++i) pr[lane * DL + i] = ag[i];
            if (lane == 0) {
                pr[D] = mg;
                pr[D + 1] = lg;
            }
        }
    }
}

// out [rows, D] from `split` partial rows [D sums, max, sum] each (sycl_be::attention_combine's layout). A workgroup of
// four waves a row: the threads take the splits for the max, the weights and the denominator, then (dim, split
// quarter) pairs, each summing its share of the column with the weights from LDS; the quarters add up in LDS.
constexpr int kMaxSplit = 256;

__global__ __launch_bounds__(256) void attention_combine_rows(const float* part, float* out, int split, int64_t D) {
    __shared__ float weight[kMaxSplit];
    __shared__ float red[256];
    const int64_t r = blockIdx.x;
    const int tid = threadIdx.x;
    const float* pr = part + r * split * (D + 2);
    float mx = -INFINITY;
    for (int s = tid; s < split; s += 256) mx = fmaxf(mx, pr[s * (D + 2) + D]);
    mx = group_reduce<64, OpMax>(mx);
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float den = 0.0f;
    for (int s = tid; s < split; s += 256) {
        const float ms = pr[s * (D + 2) + D];
        const float w = ms == -INFINITY ? 0.0f : __expf(ms - mx);
        weight[s] = w;
        den += pr[s * (D + 2) + D + 1] * w;
    }
    den = group_reduce<64, OpSum>(den);
    if ((tid & 63) == 0) red[tid >> 6] = den;
    __syncthreads();
    den = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = 1.0f / den;
    __syncthreads();
    // Dims in chunks of 64: thread (d, quarter) sums splits quarter, quarter + 4, ...
    const int dl = tid & 63, quarter = tid >> 6;
    for (int64_t d0 = 0; d0 < D; d0 += 64) {
        const int64_t d = d0 + dl;
        float acc = 0.0f;
        if (d < D) {
            // eight loads in flight before the first is used
            for (int s0 = quarter; s0 < split; s0 += 32) {
                float v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int s = s0 + 4 * u;
                    v[u] = s < split ? pr[s * (D + 2) + d] : 0.0f;
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int s = s0 + 4 * u;
                    acc += s < split ? v[u] * weight[s] : 0.0f;
                }
            }
        }
        red[tid] = acc;
        __syncthreads();
        if (quarter == 0 && d < D) out[r * D + d] = ((red[dl] + red[64 + dl]) + (red[128 + dl] + red[192 + dl])) * inv;
        __syncthreads();
    }
}

template <int G, int D>
void launch_rows(hipStream_t s, const AttnArgs& a) {
    const dim3 grid(static_cast<unsigned>(a.split), static_cast<unsigned>(a.tokens * a.kv_heads));
    attention_i8_rows<G, D><<<grid, 64 * kWaves, 0, s>>>(a, a.q);
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

}  // namespace
}  // namespace xs_hip

using namespace xs_hip;

extern "C" {

int64_t xs_hip_attention_i8_split(int64_t tokens, int64_t kv_heads, int64_t kv_len) {
    if (tokens <= 0 || kv_heads <= 0 || kv_len <= 0) return 1;
    // Two workgroups (of four waves) for every CU, each with at least 256 keys.
    const int64_t groups = tokens * kv_heads;
    int64_t split = (2 * static_cast<int64_t>(device_cus()) + groups - 1) / groups;
    const int64_t by_len = kv_len / 256;
    if (split > by_len) split = by_len;
    if (split > kMaxSplit) split = kMaxSplit;
    return split < 1 ? 1 : split;
}

size_t xs_hip_attention_i8_scratch(int64_t tokens, int64_t q_heads, int64_t head_dim, int64_t split) {
    if (split <= 1 || tokens <= 0 || q_heads <= 0 || head_dim <= 0) return 0;
    return static_cast<size_t>(tokens * q_heads * split * (head_dim + 2)) * sizeof(float);
}

int xs_hip_attention_i8(void* stream, const float* q, const void* k_codes, const void* k_scales, const void* v_codes,
                        const void* v_scales, float* out, int64_t tokens, int64_t q_heads, int64_t kv_heads,
                        int64_t head_dim, int64_t kv_len, float scale, float softcap, int64_t window, int causal,
                        int64_t split, void* scratch) {
    const char* what = "xs_hip_attention_i8";
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
    if (!aligned16(q) || !aligned16(out) || !aligned16(k_codes) || !aligned16(v_codes) || head_dim % 16 != 0 ||
        (split > 1 && reinterpret_cast<uintptr_t>(scratch) % 16 != 0))
        return fail(XS_HIP_EINVAL, std::string(what) + ": q, out, codes and scratch must be 16-byte aligned and "
                                                       "head_dim a multiple of 16");
    AttnArgs a{q, static_cast<const int8_t*>(k_codes), static_cast<const float*>(k_scales),
               static_cast<const int8_t*>(v_codes), static_cast<const float*>(v_scales),
               out, split > 1 ? static_cast<float*>(scratch) : nullptr, tokens, q_heads, kv_heads, head_dim, kv_len,
               window, scale, softcap, causal ? 1 : 0, static_cast<int>(split)};
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
    attention_combine_rows<<<static_cast<unsigned>(tokens * q_heads), 256, 0, s>>>(
        static_cast<const float*>(scratch), out, static_cast<int>(split), head_dim);
    return check_launch("xs_hip_attention_i8 (combine)");
}

}  // extern "C"
