// Rotate-half (NeoX) RoPE for gfx950.
//
// Semantics: cpu_ref::rope (reference src/backend/cpu_ref/ops.cpp:343-399), spec graph.h Rope (src/graph/graph.h:
// 119-127): for a pair (c1, c2 = c1 + W/2) of a section of width W, angle = double(pos) * double(inv_freq[i]),
// c, s = cos, sin(angle) in f64, y1 = fl32(x1 * c - x2 * s), y2 = fl32(x2 * c + x1 * s) with the products and sums in
// f64; channels past `rotary` pass through. Axial positions [T, S] rotate section s by positions[:, s]; with pair_axes
// one section whose pair i reads positions[:, pair_axes[i]]. Launcher replaced: sycl_be::rope
// (src/backend/sycl/sycl_kernels.h:114-116, sycl_kernels.cpp:1678-1717), which uses an f32 angle; this kernel keeps the
// reference CPU path's f64 angle, so its outputs round from the same f64 values cpu-ref computes.
//
// Two kernels. The row-contiguous kernel (rope_rows_kernel, below) takes the common shapes -- rotary == dim, one
// section or pair axes, rows of 8, 16 or 32 128-bit vectors: a block's loads and stores are those of a plain copy over
// whole tokens of Q and K, and partner lanes swap half-rows through DPP. The per-pair kernel (rope_kernel) takes every
// other shape (sections, partial rotary, odd widths): a block of 256 threads takes a tile of TT tokens (about four
// units of work per thread). It first fills an LDS table of (cos, sin) in f64 for the tile's TT x pairs entries -- one
// sincos per (token, pair), shared by every head of the token; one f64 pair of padding every 8 entries spreads the 8
// entries a wave reads at once over distinct LDS banks. Then thread t walks the tile's units t, t + 256, ... -- a unit
// is (token, head, VEC consecutive pairs): one 128-bit load of x1 and one of x2, the rotation, two stores. The rotation
// is an f64 FMA of the exactly widened inputs, rounded to f32 and then to y's dtype, as cpu-ref's f64 expression is.
// Measured on MI355X at the Q+K shape of 8192 tokens x (32 + 8) heads x 128, f16: the per-pair kernel 33.3 us, the
// row-contiguous one 29.6 us, a plain copy of the same bytes 27.5 us.
#include <cmath>

#include "common.h"

namespace xs_hip {
namespace {

struct RopeArgs {
    const void* x;
    const void* pos;
    const float* inv_freq;
    void* y;
    const int32_t* pair_axes;
    int64_t tokens, heads, dim, rotary, sections;
    int tile_tokens;
    // An optional second tensor of the same tokens (K beside Q): x2 / y2 [tokens, heads2, dim]; heads2 = 0 for none.
    const void* x2;
    void* y2;
    int64_t heads2;
};

// The element offset of (token t, head h) and the tensor it lies in: heads [0, heads) are x / y, heads
// [heads, heads + heads2) the second tensor.
template <typename SX, typename SY>
__device__ __forceinline__ int64_t head_at(const RopeArgs& a, int64_t t, int h, const SX*& x, SY*& y) {
    if (h < a.heads) {
        x = static_cast<const SX*>(a.x);
        y = static_cast<SY*>(a.y);
        return (t * a.heads + h) * a.dim;
    }
    x = static_cast<const SX*>(a.x2);
    y = static_cast<SY*>(a.y2);
    return (t * a.heads2 + (h - a.heads)) * a.dim;
}

template <typename I>
__device__ __forceinline__ int64_t pos_at(const void* p, int64_t i) {
    return static_cast<int64_t>(static_cast<const I*>(p)[i]);
}

// Stores N consecutive outputs (N = 1, 4 or 8) of type T.
template <typename T, int N>
__device__ __forceinline__ void store_n(typename T::storage* p, const float* f) {
    if constexpr (N == 1) {
        p[0] = T::store(f[0]);
    } else if constexpr (N * sizeof(typename T::storage) == 16) {
        st128(p, pack<T>(f));
    } else if constexpr (N * sizeof(typename T::storage) == 32) {
        st128(p, pack<T>(f));
        st128(p + 16 / sizeof(typename T::storage), pack<T>(f + 16 / sizeof(typename T::storage)));
    } else {  // 4 x 16-bit = 8 bytes
        uint2 v;
        v.x = pack2<T>(f[0], f[1]);
        v.y = pack2<T>(f[2], f[3]);
        *reinterpret_cast<uint2*>(p) = v;
    }
}

template <typename T, int N>
__device__ __forceinline__ void load_n(const typename T::storage* p, float* f) {
    if constexpr (N == 1) {
        f[0] = T::load(p[0]);
    } else {
        static_assert(N * sizeof(typename T::storage) == 16, "one 128-bit vector");
        unpack<T>(ld128_nt(p), f);
    }
}

constexpr int kMaxTableEntries = 1024;  // (cos, sin) f64 pairs per block, before padding: 18 KiB of LDS
constexpr int kTableSlots = kMaxTableEntries + kMaxTableEntries / 8;

__device__ __forceinline__ int table_slot(int e) { return e + (e >> 3); }

// y1 = x1 c - x2 s, y2 = x2 c + x1 s in f64, each rounded to f32.
template <int VEC>
__device__ __forceinline__ void rotate(const float* x1, const float* x2, const double2* cs, float* y1, float* y2) {
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        const double d1 = x1[k], d2 = x2[k];
        y1[k] = static_cast<float>(fma(d1, cs[k].x, -(d2 * cs[k].y)));
        y2[k] = static_cast<float>(fma(d2, cs[k].x, d1 * cs[k].y));
    }
}

template <typename TX, typename TY, typename I, int VEC>
__global__ __launch_bounds__(kBlock) void rope_kernel(RopeArgs a, FastDiv32 pv_div) {
    using SX = typename TX::storage;
    using SY = typename TY::storage;
    __shared__ double2 table[kTableSlots];

    const int64_t pairs = a.rotary / 2;
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * a.tile_tokens;
    const int tt_n = static_cast<int>(a.tokens - t0 < a.tile_tokens ? a.tokens - t0 : a.tile_tokens);
    const bool axes = a.pair_axes != nullptr;
    const int64_t width = axes ? a.rotary : a.rotary / a.sections;  // section width
    const int64_t half = width / 2;
    const int heads = static_cast<int>(a.heads + a.heads2);
    const int pv_per_head = static_cast<int>(pairs / VEC);
    const int upt = heads * pv_per_head;  // rotation units per token

    // The thread's first unit is loaded before the table is built, so its HBM latency overlaps the sincos work.
    int tt = threadIdx.x / upt;
    int slot = threadIdx.x - tt * upt;
    float x1[VEC], x2[VEC];
    const SX* x = nullptr;
    SY* y = nullptr;
    int64_t base = 0;
    int p0 = 0;
    auto locate = [&]() {
        const int h = static_cast<int>(pv_div.div(static_cast<uint32_t>(slot)));
        p0 = (slot - h * pv_per_head) * VEC;
        int64_t c1 = p0;
        if (!axes) {
            const int64_t sec = p0 / half;
            c1 = sec * width + (p0 - sec * half);
        }
        base = head_at(a, t0 + tt, h, x, y) + c1;
    };
    if (tt < tt_n) {
        locate();
        load_n<TX, VEC>(x + base, x1);
        load_n<TX, VEC>(x + base + half, x2);
    }

    // (cos, sin) of every (token, pair) of the tile.
    const int entries = tt_n * static_cast<int>(pairs);
    for (int e = threadIdx.x; e < entries; e += kBlock) {
        const int te = e / static_cast<int>(pairs);
        const int64_t p = e - static_cast<int64_t>(te) * pairs;
        int64_t sec, i;
        if (axes) {
            // Axes outside [0, sections) are a caller error the host cannot see in device memory; clamp so the read
            // stays in bounds.
            sec = a.pair_axes[p];
            sec = sec < 0 ? 0 : (sec >= a.sections ? a.sections - 1 : sec);
            i = p;
        } else {
            sec = p / half;
            i = p - sec * half;
        }
        const double pos = static_cast<double>(pos_at<I>(a.pos, (t0 + te) * a.sections + sec));
        const double angle = pos * static_cast<double>(a.inv_freq[i]);
        double sn, cs;
        sincos(angle, &sn, &cs);
        table[table_slot(e)] = make_double2(cs, sn);
    }
    __syncthreads();

    // Thread t takes units t, t + kBlock, ... of the tile; (token, slot) of the next unit follows from the last by
    // adding kBlock to the slot and carrying whole tokens, so no unit needs a division.
    const int carry_t = kBlock / upt, carry_s = kBlock - carry_t * upt;
    bool first = true;
    for (; tt < tt_n;) {
        if (!first) {
            locate();
            load_n<TX, VEC>(x + base, x1);
            load_n<TX, VEC>(x + base + half, x2);
        }
        first = false;
        float y1[VEC], y2[VEC];
        double2 cs[VEC];
#pragma unroll
        for (int k = 0; k < VEC; ++k) cs[k] = table[table_slot(tt * static_cast<int>(pairs) + p0 + k)];
        rotate<VEC>(x1, x2, cs, y1, y2);
        store_n<TY, VEC>(y + base, y1);
        store_n<TY, VEC>(y + base + half, y2);
        tt += carry_t;
        slot += carry_s;
        if (slot >= upt) {
            slot -= upt;
            ++tt;
        }
    }

    // Channels past the rotary dims pass through (unless y is x).
    if (a.rotary < a.dim) {
        const int64_t rest = a.dim - a.rotary;
        const int64_t units = static_cast<int64_t>(tt_n) * heads * rest;
        for (int64_t u = threadIdx.x; u < units; u += kBlock) {
            const int64_t th = u / rest;
            const int64_t tu = th / heads;
            const int hu = static_cast<int>(th - tu * heads);
            const SX* xp;
            SY* yp;
            const int64_t at = head_at(a, t0 + tu, hu, xp, yp) + a.rotary + (u - th * rest);
            if (static_cast<const void*>(xp) != static_cast<const void*>(yp)) yp[at] = TY::store(TX::load(xp[at]));
        }
    }
}

// ---- Row-contiguous kernel (rotary == dim, one section or pair axes, a row of R = dim / VEC 128-bit vectors with R
// 8, 16 or 32) --------------------------------------------------------------------------------------------
//
// A block takes TT whole tokens: the rows of those tokens in x (heads) and then in x2 (heads2), which are two contiguous
// runs of memory. Thread t reads vectors t, t + 256, ... of that run with one 128-bit load each -- the access pattern of
// a plain copy, every wave instruction covering 1 KiB of consecutive bytes. Since 256 is a multiple of R, a thread's
// vector sits at the same place v = t % R in every row it visits: lanes with v < R/2 hold x1 (the first half of the
// row), and the partner lane t ^ (R/2) holds the x2 of the same pairs. The partners split the work: the "lo" lane
// rotates the first VEC/2 pairs of the vector and the "hi" lane the last VEC/2, each after receiving the other's two
// dwords of input, and they swap two dwords of results back so each stores its own vector. So each lane reads VEC/2
// (cos, sin) entries from the LDS table per vector, and the rotation and roundings are the same f64 expression as the
// kernel above.
template <int M>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v) {
    if constexpr (M == 8) {
        // row_ror:8 within each 16-lane row is lane ^ 8.
        return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(v), static_cast<int>(v), 0x128, 0xF,
                                                                 0xF, false));
    } else if constexpr (M == 1) {
        return static_cast<uint32_t>(dpp_i<dpp::kQuadXor1>(static_cast<int>(v)));
    } else if constexpr (M == 2) {
        return static_cast<uint32_t>(dpp_i<dpp::kQuadXor2>(static_cast<int>(v)));
    } else {
        return static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), M, 64));
    }
}

// Lanes selected by BankMask (4 lanes a bank, 4 banks a 16-lane row) take `src` of lane ^ 8; the others keep `own`.
template <int BankMask>
__device__ __forceinline__ uint32_t dpp_merge(uint32_t own, uint32_t src) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(static_cast<int>(own), static_cast<int>(src), 0x128, 0xF, BankMask, false));
}

struct RowArgs {
    const void* x;
    void* y;
    const void* x2;
    void* y2;
    const void* pos;
    const float* inv_freq;
    const int32_t* pair_axes;
    int64_t tokens, sections;
    int heads, heads2, pairs;  // pairs = dim / 2
    int tile_tokens;
    FastDiv32 row_vecs_a, row_vecs_b;  // dividers by heads * R and heads2 * R (vectors per token of each tensor)
};

// Threads of a row-kernel workgroup (64 and 128 measured slower on MI355X at config 3's shape).
constexpr int kRowBlock = 256;

template <typename TX, typename TY, typename I, int R, int NV>
__global__ __launch_bounds__(kRowBlock) void rope_rows_kernel(RowArgs a) {
    using SX = typename TX::storage;
    using SY = typename TY::storage;
    constexpr int VEC = vec_elems<TX>();
    constexpr int H = VEC / 2;                      // pairs each partner rotates
    constexpr int YW = H * sizeof(SY) / 4;          // dwords of H outputs
    constexpr int YB = VEC * sizeof(SY);            // bytes of one output vector: 8, 16 or 32
    static_assert(R >= 2 && R <= 64 && (R & (R - 1)) == 0, "row of a power-of-two count of vectors");
    __shared__ double2 table[kTableSlots];

    const int t = threadIdx.x;
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * a.tile_tokens;
    const int tt_n = static_cast<int>(a.tokens - t0 < a.tile_tokens ? a.tokens - t0 : a.tile_tokens);
    const int na = tt_n * a.heads * R;             // vectors of the tile in x
    const int n = na + tt_n * a.heads2 * R;         // and in x2
    const int v = t & (R - 1);
    const bool hi = v >= R / 2;
    const int pbase = (v & (R / 2 - 1)) * VEC + (hi ? H : 0);  // first pair this lane rotates

    const SX* xa = static_cast<const SX*>(a.x) + t0 * a.heads * R * VEC;
    const SX* xb = static_cast<const SX*>(a.x2) + t0 * a.heads2 * R * VEC;
    // Every load is issued, those past the tile re-reading its last vector, so no branch separates them.
    u32x4 raw[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int j = min(t + k * kRowBlock, n - 1);
        raw[k] = ld128_nt(j < na ? xa + static_cast<int64_t>(j) * VEC : xb + static_cast<int64_t>(j - na) * VEC);
    }

    // (cos, sin) of every (token, pair) of the tile, as the kernel above builds it.
    const int entries = tt_n * a.pairs;
    for (int e = t; e < entries; e += kRowBlock) {
        const int te = e / a.pairs;
        const int p = e - te * a.pairs;
        int64_t sec = 0;
        if (a.pair_axes != nullptr) {
            sec = a.pair_axes[p];
            sec = sec < 0 ? 0 : (sec >= a.sections ? a.sections - 1 : sec);
        }
        const double pos = static_cast<double>(pos_at<I>(a.pos, (t0 + te) * a.sections + sec));
        const double angle = pos * static_cast<double>(a.inv_freq[p]);
        double sn, cs;
        sincos(angle, &sn, &cs);
        table[table_slot(e)] = make_double2(cs, sn);
    }
    __syncthreads();

    SY* ya = static_cast<SY*>(a.y) + t0 * a.heads * R * VEC;
    SY* yb = static_cast<SY*>(a.y2) + t0 * a.heads2 * R * VEC;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int j = t + k * kRowBlock;
        if (j >= n) break;  // rows are whole, so a lane and its partner leave together
        const int tl = static_cast<int>(j < na ? a.row_vecs_a.div(static_cast<uint32_t>(j))
                                               : a.row_vecs_b.div(static_cast<uint32_t>(j - na)));
        // lo keeps x1 of pairs [0, H) and receives x2 of them; hi keeps x2 of [H, VEC) and receives x1 of them.
        u32x4 own1, own2;  // x1 and x2 of this lane's H pairs, in the first two dwords
        if constexpr (R == 16) {
            // The partner is lane ^ 8 in the lane's 16-lane row: row_ror:8, written only into the lanes that take
            // the partner's word (bank_mask 0xC: lanes 8..15 of each row, the hi lanes; 0x3: the lo lanes).
            own1[0] = dpp_merge<0xC>(raw[k][0], raw[k][2]);
            own1[1] = dpp_merge<0xC>(raw[k][1], raw[k][3]);
            own2[0] = dpp_merge<0x3>(raw[k][2], raw[k][0]);
            own2[1] = dpp_merge<0x3>(raw[k][3], raw[k][1]);
        } else {
            const uint32_t s0 = xor_lane<R / 2>(hi ? raw[k][0] : raw[k][2]);
            const uint32_t s1 = xor_lane<R / 2>(hi ? raw[k][1] : raw[k][3]);
            own1[0] = hi ? s0 : raw[k][0];
            own1[1] = hi ? s1 : raw[k][1];
            own2[0] = hi ? raw[k][2] : s0;
            own2[1] = hi ? raw[k][3] : s1;
        }
        own1[2] = own1[3] = own2[2] = own2[3] = 0;
        float x1[VEC], x2[VEC];
        unpack<TX>(own1, x1);
        unpack<TX>(own2, x2);
        float y1[H], y2[H];
        // The H entries share one group of 8 (pairs and pbase are multiples of H, H <= 4), so their slots are
        // consecutive.
        const double2* cs_row = table + table_slot(tl * a.pairs + pbase);
#pragma unroll
        for (int i = 0; i < H; ++i) {
            const double2 cs = cs_row[i];
            const double d1 = x1[i], d2 = x2[i];
            y1[i] = static_cast<float>(fma(d1, cs.x, -(d2 * cs.y)));
            y2[i] = static_cast<float>(fma(d2, cs.x, d1 * cs.y));
        }
        // Narrow this lane's H results of each half; lo stores y1 of all VEC pairs, hi y2.
        uint32_t p1[YW], p2[YW];
        if constexpr (sizeof(SY) == 4) {
#pragma unroll
            for (int i = 0; i < H; ++i) {
                p1[i] = __float_as_uint(y1[i]);
                p2[i] = __float_as_uint(y2[i]);
            }
        } else {
#pragma unroll
            for (int i = 0; i < YW; ++i) {
                p1[i] = pack2<TY>(y1[2 * i], y1[2 * i + 1]);
                p2[i] = pack2<TY>(y2[2 * i], y2[2 * i + 1]);
            }
        }
        uint32_t out[2 * YW];
#pragma unroll
        for (int i = 0; i < YW; ++i) {
            if constexpr (R == 16) {
                out[i] = dpp_merge<0xC>(p1[i], p2[i]);       // hi takes lo's y2
                out[YW + i] = dpp_merge<0x3>(p2[i], p1[i]);  // lo takes hi's y1
            } else {
                const uint32_t got = xor_lane<R / 2>(hi ? p1[i] : p2[i]);  // lo sends y2, hi sends y1
                out[i] = hi ? got : p1[i];
                out[YW + i] = hi ? p2[i] : got;
            }
        }
        SY* dst = (j < na ? ya + static_cast<int64_t>(j) * VEC : yb + static_cast<int64_t>(j - na) * VEC);
        if constexpr (YB == 8) {
            typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
            u32x2 w;
            w[0] = out[0];
            w[1] = out[1];
            __builtin_nontemporal_store(w, reinterpret_cast<u32x2*>(dst));
        } else {
#pragma unroll
            for (int q = 0; q < YB / 16; ++q) {
                u32x4 w;
                w[0] = out[4 * q];
                w[1] = out[4 * q + 1];
                w[2] = out[4 * q + 2];
                w[3] = out[4 * q + 3];
                st128_nt(dst + q * (16 / sizeof(SY)), w);
            }
        }
        // Keeps the scheduler from hoisting every vector's table reads ahead of the first store, which would hold
        // NV vectors' worth of f64 (cos, sin) in registers at once.
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Vectors per thread the row kernel is instantiated for, and the tile it aims at (vectors per block).
constexpr int kRowMaxNV = 8;
constexpr int kRowTargetVectors = 2 * kRowBlock;  // one token of Q+K at config 3 (measured best against 6x)

template <typename TX, typename TY, typename I, int R>
int launch_rows_nv(hipStream_t s, const RowArgs& a, int nv, unsigned grid) {
    // Instantiated for an even count of vectors per thread (the last one idles when the tile needs an odd count).
    switch ((nv + 1) / 2) {
        case 1: rope_rows_kernel<TX, TY, I, R, 2><<<grid, kRowBlock, 0, s>>>(a); break;
        case 2: rope_rows_kernel<TX, TY, I, R, 4><<<grid, kRowBlock, 0, s>>>(a); break;
        case 3: rope_rows_kernel<TX, TY, I, R, 6><<<grid, kRowBlock, 0, s>>>(a); break;
        default: rope_rows_kernel<TX, TY, I, R, 8><<<grid, kRowBlock, 0, s>>>(a); break;
    }
    return check_launch("xs_hip_rope");
}

// Launches the row kernel when the shape suits it; returns -1 (nothing launched) otherwise.
template <typename TX, typename TY, typename I>
int try_launch_rows(hipStream_t s, const RopeArgs& a) {
    constexpr int VEC = vec_elems<TX>();
    if (a.rotary != a.dim || (a.sections != 1 && a.pair_axes == nullptr) || a.dim % VEC != 0) return -1;
    const int64_t r = a.dim / VEC;
    if (r != 8 && r != 16 && r != 32) return -1;  // head dims 64 / 128 / 256 at 16 bits, 32 / 64 / 128 at 32 bits
    if (!aligned16(a.x) || !aligned16(a.y) || (a.heads2 > 0 && (!aligned16(a.x2) || !aligned16(a.y2)))) return -1;
    const int64_t per_token = (a.heads + a.heads2) * r;  // vectors
    if (per_token > static_cast<int64_t>(kRowMaxNV) * kRowBlock) return -1;
    int64_t tt = kRowTargetVectors / per_token;
    if (tt < 1) tt = 1;
    const int64_t pairs = a.dim / 2;
    if (tt * pairs > kMaxTableEntries) tt = kMaxTableEntries / pairs;
    if (tt < 1) return -1;
    if (tt > a.tokens) tt = a.tokens;
    const int nv = static_cast<int>((tt * per_token + kRowBlock - 1) / kRowBlock);
    RowArgs ra;
    ra.x = a.x;
    ra.y = a.y;
    ra.x2 = a.heads2 > 0 ? a.x2 : a.x;
    ra.y2 = a.heads2 > 0 ? a.y2 : a.y;
    ra.pos = a.pos;
    ra.inv_freq = a.inv_freq;
    ra.pair_axes = a.pair_axes;
    ra.tokens = a.tokens;
    ra.sections = a.sections;
    ra.heads = static_cast<int>(a.heads);
    ra.heads2 = static_cast<int>(a.heads2);
    ra.pairs = static_cast<int>(pairs);
    ra.tile_tokens = static_cast<int>(tt);
    ra.row_vecs_a = FastDiv32(static_cast<uint32_t>(a.heads * r));
    ra.row_vecs_b = FastDiv32(static_cast<uint32_t>(a.heads2 > 0 ? a.heads2 * r : 1));
    const unsigned grid = static_cast<unsigned>((a.tokens + tt - 1) / tt);
    switch (r) {
        case 8: return launch_rows_nv<TX, TY, I, 8>(s, ra, nv, grid);
        case 16: return launch_rows_nv<TX, TY, I, 16>(s, ra, nv, grid);
        default: return launch_rows_nv<TX, TY, I, 32>(s, ra, nv, grid);
    }
}

template <typename TX, typename TY, typename I>
int launch_rope(hipStream_t s, RopeArgs a) {
    const int rows_rc = try_launch_rows<TX, TY, I>(s, a);
    if (rows_rc >= 0) return rows_rc;
    constexpr int VEC = vec_elems<TX>();
    const int64_t pairs = a.rotary / 2;
    const bool axes = a.pair_axes != nullptr;
    const int64_t half = axes ? pairs : (a.rotary / a.sections) / 2;
    const bool vec = half % VEC == 0 && a.dim % VEC == 0 && aligned16(a.x) && aligned16(a.y) &&
                     (a.heads2 == 0 || (aligned16(a.x2) && aligned16(a.y2)));
    const int64_t pv = pairs / (vec ? VEC : 1);
    const int64_t upt = (a.heads + a.heads2) * pv;  // rotation units per token
    // Tile: about four units per thread (measured best on MI355X against two and eight), within the LDS table.
    int64_t tt = (4 * kBlock + upt - 1) / upt;
    const int64_t max_tt = pairs > 0 ? kMaxTableEntries / pairs : 64;
    if (tt > max_tt) tt = max_tt;
    if (tt < 1) tt = 1;
    a.tile_tokens = static_cast<int>(tt);
    const unsigned grid = static_cast<unsigned>((a.tokens + tt - 1) / tt);
    const FastDiv32 pv_div(static_cast<uint32_t>(pv));
    if (vec) rope_kernel<TX, TY, I, VEC><<<grid, kBlock, 0, s>>>(a, pv_div);
    else rope_kernel<TX, TY, I, 1><<<grid, kBlock, 0, s>>>(a, pv_div);
    return check_launch("xs_hip_rope");
}

template <typename TX, typename TY>
int rope_pos(hipStream_t s, const RopeArgs& a, xs_dtype pos_dtype) {
    switch (pos_dtype) {
        case XS_I32: return launch_rope<TX, TY, int32_t>(s, a);
        case XS_I64: return launch_rope<TX, TY, int64_t>(s, a);
        default: return fail(XS_HIP_EINVAL, std::string("xs_hip_rope: positions must be i32 or i64, got ") + dtype_name(pos_dtype));
    }
}

template <typename TX>
int rope_y(hipStream_t s, const RopeArgs& a, xs_dtype pos_dtype, xs_dtype y_dtype) {
    switch (y_dtype) {
        case XS_F32: return rope_pos<TX, F32>(s, a, pos_dtype);
        case XS_F16: return rope_pos<TX, F16>(s, a, pos_dtype);
        case XS_BF16: return rope_pos<TX, BF16>(s, a, pos_dtype);
        default: return fail(XS_HIP_EINVAL, std::string("xs_hip_rope: y must be f32, f16 or bf16, got ") + dtype_name(y_dtype));
    }
}

std::string i2s(int64_t v) { return std::to_string(v); }

}  // namespace
}  // namespace xs_hip

using namespace xs_hip;

namespace xs_hip {
namespace {

int check_overlap(const void* x, const void* y, int64_t n, xs_dtype xt, xs_dtype yt, const char* what) {
    if (x == y) return XS_HIP_OK;
    const int esx = float_size(xt), esy = float_size(yt);
    const char* xb = static_cast<const char*>(x);
    const char* yb = static_cast<const char*>(y);
    if (esx > 0 && esy > 0 && xb < yb + n * esy && yb < xb + n * esx)
        return fail(XS_HIP_EINVAL, std::string(what) + ": y overlaps x without being x");
    return XS_HIP_OK;
}

int rope_common(void* stream, xs_dtype x_dtype, const void* x, xs_dtype pos_dtype, const void* positions,
                const float* inv_freq, xs_dtype y_dtype, void* y, int64_t tokens, int64_t heads, int64_t dim,
                int64_t rotary, int64_t sections, const int32_t* pair_axes, const void* x2, void* y2, int64_t heads2,
                const char* what) {
    if (rotary == 0) rotary = dim;
    if (tokens < 0 || heads <= 0 || heads2 < 0 || dim <= 0 || rotary < 0 || rotary > dim || sections <= 0)
        return fail(XS_HIP_EINVAL, std::string(what) + ": x [" + i2s(tokens) + ", " + i2s(heads) + ", " + i2s(dim) +
                                       "], rotary " + i2s(rotary) + ", sections " + i2s(sections));
    if (pair_axes == nullptr && (rotary % (2 * sections) != 0))
        return fail(XS_HIP_EINVAL, std::string(what) + ": rotary dims " + i2s(rotary) + " do not split into " +
                                       i2s(sections) + " sections of pairs");
    if (pair_axes != nullptr && rotary % 2 != 0)
        return fail(XS_HIP_EINVAL, std::string(what) + ": rotary dims " + i2s(rotary) + " are odd");
    if (tokens == 0) return XS_HIP_OK;
    if (x == nullptr || positions == nullptr || inv_freq == nullptr || y == nullptr ||
        (heads2 > 0 && (x2 == nullptr || y2 == nullptr)))
        return fail(XS_HIP_EINVAL, std::string(what) + ": null buffer");
    if (rotary / 2 > kMaxTableEntries)
        return fail(XS_HIP_EUNSUPPORTED, std::string(what) + ": " + i2s(rotary / 2) + " pairs per head exceed " +
                                             i2s(kMaxTableEntries));
    if (tokens > 0x7fffffffLL || (heads + heads2) * (rotary / 2) > (int64_t{1} << 24))
        return fail(XS_HIP_EUNSUPPORTED, std::string(what) + ": shape too large");
    int rc = check_overlap(x, y, tokens * heads * dim, x_dtype, y_dtype, what);
    if (rc == XS_HIP_OK && heads2 > 0) rc = check_overlap(x2, y2, tokens * heads2 * dim, x_dtype, y_dtype, what);
    if (rc != XS_HIP_OK) return rc;
    const RopeArgs a{x, positions, inv_freq, y, pair_axes, tokens, heads, dim, rotary, sections, 1, x2, y2, heads2};
    const hipStream_t s = as_stream(stream);
    switch (x_dtype) {
        case XS_F32: return rope_y<F32>(s, a, pos_dtype, y_dtype);
        case XS_F16: return rope_y<F16>(s, a, pos_dtype, y_dtype);
        case XS_BF16: return rope_y<BF16>(s, a, pos_dtype, y_dtype);
        default:
            return fail(XS_HIP_EINVAL, std::string(what) + ": x must be f32, f16 or bf16, got " + dtype_name(x_dtype));
    }
}

}  // namespace
}  // namespace xs_hip

extern "C" {

int xs_hip_rope(void* stream, xs_dtype x_dtype, const void* x, xs_dtype pos_dtype, const void* positions,
                const float* inv_freq, xs_dtype y_dtype, void* y, int64_t tokens, int64_t heads, int64_t dim,
                int64_t rotary, int64_t sections, const int32_t* pair_axes) {
    return rope_common(stream, x_dtype, x, pos_dtype, positions, inv_freq, y_dtype, y, tokens, heads, dim, rotary,
                       sections, pair_axes, nullptr, nullptr, 0, "xs_hip_rope");
}

int xs_hip_rope2(void* stream, xs_dtype x_dtype, const void* xa, void* ya, int64_t heads_a, const void* xb, void* yb,
                 int64_t heads_b, xs_dtype pos_dtype, const void* positions, const float* inv_freq, xs_dtype y_dtype,
                 int64_t tokens, int64_t dim, int64_t rotary, int64_t sections, const int32_t* pair_axes) {
    if (heads_b <= 0) return fail(XS_HIP_EINVAL, "xs_hip_rope2: the second tensor has no heads");
    return rope_common(stream, x_dtype, xa, pos_dtype, positions, inv_freq, y_dtype, ya, tokens, heads_a, dim, rotary,
                       sections, pair_axes, xb, yb, heads_b, "xs_hip_rope2");
}

}  // extern "C"
