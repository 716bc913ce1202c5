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
// Layout: one workgroup of four waves per (token, KV head, key split). The G query heads sharing the KV head are
// handled together, so each key and value row is read once for all of them. L lanes cover one key's head_dim
// (DPL = head_dim / L codes a lane: one 16- or 8-byte load of key codes and one of value codes), so a wave works on
// 64 / L keys at once; each lane group keeps four keys' loads in flight. Scores: each lane's partial dot product in f32, reduced over its L lanes by
// DPP; times the key's scale and the softmax scale. An online softmax per head (the running max moves, and the
// accumulator is rescaled, only when a larger score arrives) accumulates p * v_scale * codes in f32. At the end the
// wave's key groups merge their (max, sum, accumulator) by shuffles and the four waves through LDS. With one split the wave writes the output; with
// several it writes [head_dim partial sums, max, sum] rows that xs_hip_attention_combine merges (flash decoding).
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

template <int DPL>
using Codes = typename std::conditional<DPL == 16, u32x4, uint64_t>::type;

template <int DPL>
__device__ __forceinline__ Codes<DPL> load_codes(const int8_t* p) {
    if constexpr (DPL == 16) return ld128_nt(p);
    else return __builtin_nontemporal_load(reinterpret_cast<const uint64_t*>(p));
}

// Code i of a lane's DPL codes, as f32.
template <int DPL>
__device__ __forceinline__ float code_at(const Codes<DPL>& c, int i) {
    uint32_t w;
    if constexpr (DPL == 16) w = c[i >> 2];
    else w = static_cast<uint32_t>(c >> (32 * (i >> 2)));
    return static_cast<float>(static_cast<int8_t>((w >> (8 * (i & 3))) & 0xffu));
}

constexpr int kWaves = 4;  // waves a workgroup; they split the workgroup's keys and merge in LDS
constexpr int kUnroll = 4;  // keys a lane group has in flight

// Merges (m, l, acc) of another key set into this one: the online-softmax combine.
template <int DPL>
__device__ __forceinline__ void merge(float& m, float& l, float* acc, float mo, float lo, const float* acco) {
    const float mm = fmaxf(m, mo);
    const float ca = m == -INFINITY ? 0.0f : __expf(m - mm);  // an empty side (max -inf) contributes nothing
    const float cb = mo == -INFINITY ? 0.0f : __expf(mo - mm);
    l = l * ca + lo * cb;
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[i] = acc[i] * ca + acco[i] * cb;
    m = mm;
}

template <int G, int DPL, int L>
__global__ __launch_bounds__(64 * kWaves) void attention_i8_rows(AttnArgs a) {
    constexpr int KG = 64 / L;        // keys a wave works on at once
    constexpr int KGB = KG * kWaves;  // ... a workgroup
    __shared__ float merge_buf[kWaves][G][L * DPL + 2];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int li = lane % L;   // which DPL codes of the row
    const int kg = lane / L;   // which key of the wave's KG
    const int64_t D = a.head_dim;
    const int64_t row = blockIdx.x;  // (t, kv head)
    const int64_t t = row / a.kv_heads;
    const int64_t kvh = row - t * a.kv_heads;
    const int s = blockIdx.y;

    int64_t first, last;
    key_range(a, t, first, last);
    const int64_t len = last >= first ? last - first + 1 : 0;
    const int64_t per = (len + a.split - 1) / a.split;
    const int64_t k0 = first + s * per;
    int64_t k1 = k0 + per - 1;
    if (k1 > last) k1 = last;

    float qv[G][DPL];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float* qp = a.q + (t * a.q_heads + kvh * G + g) * D + li * DPL;
#pragma unroll
        for (int i = 0; i < DPL; i += 4) {
            const u32x4 raw = ld128(qp + i);
#pragma unroll
            for (int w = 0; w < 4; ++w) qv[g][i + w] = __uint_as_float(raw[w]) * a.scale;
        }
    }
    float acc[G][DPL];
    float m[G], l[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.0f;
#pragma unroll
        for (int i = 0; i < DPL; ++i) acc[g][i] = 0.0f;
    }

    // Key j of this lane group: k0 + kg + wave * KG + n * KGB. Each pass loads kUnroll keys (clamped to the last one,
    // whose repeats are not used), then folds them in.
    for (int64_t jb = k0 + wave * KG + kg; jb <= k1; jb += kUnroll * KGB) {
        Codes<DPL> kc[kUnroll], vc[kUnroll];
        float ksc[kUnroll], vsc[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int64_t j = jb + u * KGB <= k1 ? jb + u * KGB : k1;
            const int64_t r = j * a.kv_heads + kvh;
            kc[u] = load_codes<DPL>(a.kc + r * D + li * DPL);
            vc[u] = load_codes<DPL>(a.vc + r * D + li * DPL);
            ksc[u] = a.ks[r];
            vsc[u] = a.vs[r];
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            if (jb + u * KGB > k1) break;  // the lane group's keys end together
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float d = 0.0f;
#pragma unroll
                for (int i = 0; i < DPL; ++i) d = fmaf(qv[g][i], code_at<DPL>(kc[u], i), d);
                d = group_reduce<L, OpSum>(d);
                float sc = d * ksc[u];
                if (a.softcap > 0.0f) sc = a.softcap * tanhf(sc / a.softcap);
                if (sc > m[g]) {
                    const float c = __expf(m[g] - sc);
                    l[g] *= c;
#pragma unroll
                    for (int i = 0; i < DPL; ++i) acc[g][i] *= c;
                    m[g] = sc;
                }
                const float p = __expf(sc - m[g]);
                l[g] += p;
                const float pv = p * vsc[u];
#pragma unroll
                for (int i = 0; i < DPL; ++i) acc[g][i] = fmaf(pv, code_at<DPL>(vc[u], i), acc[g][i]);
            }
        }
    }

    // Merge the wave's KG key groups: lanes li, li + L, ... hold the same dims of different keys.
#pragma unroll
    for (int off = L; off < 64; off <<= 1) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float ao[DPL];
#pragma unroll
            for (int i = 0; i < DPL; ++i) ao[i] = __shfl_xor(acc[g][i], off, 64);
            merge<DPL>(m[g], l[g], acc[g], __shfl_xor(m[g], off, 64), __shfl_xor(l[g], off, 64), ao);
        }
    }
    // ... then the workgroup's waves, through LDS.
    if (kg == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
#pragma unroll
            for (int i = 0; i < DPL; ++i) merge_buf[wave][g][li * DPL + i] = acc[g][i];
            if (li == 0) {
                merge_buf[wave][g][L * DPL] = m[g];
                merge_buf[wave][g][L * DPL + 1] = l[g];
            }
        }
    }
    __syncthreads();
    if (wave != 0 || kg != 0) return;  // lanes 0 .. L-1 of wave 0 finish
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float ao[DPL];
#pragma unroll
            for (int i = 0; i < DPL; ++i) ao[i] = merge_buf[w][g][li * DPL + i];
            merge<DPL>(m[g], l[g], acc[g], merge_buf[w][g][L * DPL], merge_buf[w][g][L * DPL + 1], ao);
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int64_t h = kvh * G + g;
        if (a.part == nullptr) {
            float* o = a.out + (t * a.q_heads + h) * D + li * DPL;
            const float inv = 1.0f / l[g];
#pragma unroll
            for (int i = 0; i < DPL; i += 4) {
                u32x4 w;
#pragma unroll
                for (int k = 0; k < 4; ++k) w[k] = __float_as_uint(acc[g][i + k] * inv);
                st128(o + i, w);
            }
        } else {
            float* pr = a.part + ((t * a.q_heads + h) * a.split + s) * (D + 2);
#pragma unroll
            for (int i = 0; i < DPL; ++i) pr[li * DPL + i] = acc[g][i];
            if (li == 0) {
                pr[D] = m[g];
                pr[D + 1] = l[g];
            }
        }
    }
}

// out [rows, D] from `split` partial rows [D sums, max, sum] each (sycl_be::attention_combine's layout). One wave a
// row: the lanes take the splits for the max, the weights and the denominator, then the dims, each summing its
// column over the splits with the weights from LDS.
constexpr int kMaxSplit = 256;

__global__ __launch_bounds__(64) void attention_combine_rows(const float* part, float* out, int split, int64_t D) {
    __shared__ float weight[kMaxSplit];
    const int64_t r = blockIdx.x;
    const int lane = threadIdx.x;
    const float* pr = part + r * split * (D + 2);
    float mx = -INFINITY;
    for (int s = lane; s < split; s += 64) mx = fmaxf(mx, pr[s * (D + 2) + D]);
    mx = group_reduce<64, OpMax>(mx);
    float den = 0.0f;
    for (int s = lane; s < split; s += 64) {
        const float ms = pr[s * (D + 2) + D];
        const float w = ms == -INFINITY ? 0.0f : __expf(ms - mx);
        weight[s] = w;
        den += pr[s * (D + 2) + D + 1] * w;
    }
    den = group_reduce<64, OpSum>(den);
    __syncthreads();
    const float inv = 1.0f / den;
    for (int64_t d = lane; d < D; d += 64) {
        float acc0 = 0.0f, acc1 = 0.0f, acc2 = 0.0f, acc3 = 0.0f;
        int s = 0;
        for (; s + 4 <= split; s += 4) {
            acc0 += pr[(s + 0) * (D + 2) + d] * weight[s + 0];
            acc1 += pr[(s + 1) * (D + 2) + d] * weight[s + 1];
            acc2 += pr[(s + 2) * (D + 2) + d] * weight[s + 2];
            acc3 += pr[(s + 3) * (D + 2) + d] * weight[s + 3];
        }
        for (; s < split; ++s) acc0 += pr[s * (D + 2) + d] * weight[s];
        out[r * D + d] = ((acc0 + acc1) + (acc2 + acc3)) * inv;
    }
}

template <int G, int DPL, int L>
void launch_rows(hipStream_t s, const AttnArgs& a) {
    const dim3 grid(static_cast<unsigned>(a.tokens * a.kv_heads), static_cast<unsigned>(a.split));
    attention_i8_rows<G, DPL, L><<<grid, 64 * kWaves, 0, s>>>(a);
}

// Heads per KV head G up to 4 take 16 codes a lane, more take 8 (the registers of q and the accumulator).
template <int G>
int launch_g(hipStream_t s, const AttnArgs& a) {
    constexpr int DPL = G <= 4 ? 16 : 8;
    switch (a.head_dim / DPL) {
        case 4: launch_rows<G, DPL, 4>(s, a); break;
        case 8: launch_rows<G, DPL, 8>(s, a); break;
        case 16: launch_rows<G, DPL, 16>(s, a); break;
        case 32: launch_rows<G, DPL, 32>(s, a); break;
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
    if (split > kMaxSplit || tokens * kv_heads > 0x7fffffffLL)
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
    attention_combine_rows<<<static_cast<unsigned>(tokens * q_heads), 64, 0, s>>>(
        static_cast<const float*>(scratch), out, static_cast<int>(split), head_dim);
    return check_launch("xs_hip_attention_i8 (combine)");
}

}  // extern "C"
