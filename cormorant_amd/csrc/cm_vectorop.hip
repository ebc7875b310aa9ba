// cm_vectorop.hip -- the VectorOP unit: element-wise ops with the fused activation
// (ops 0..9) and the integer softmax in row and keys-major column mode (ops 10, 11).
//
// Element-wise: one thread per 16-byte word (8 int16 lanes) of a run, so every load and
// store is a whole aligned word -- the unit's own word contract (VectorOP.h:222-236) and
// the natural HBM access of a gfx950 wavefront (64 lanes x 16 B = 1 KiB per instruction).
// The activation unit's compact tables (a few KiB) are staged in LDS per workgroup.
//
// Softmax: a row is held by 16 lanes (max and sum by DPP within the row), e looked up in a
// per-workgroup LDS table of e(max - x); column mode reads a tile of up to 64 query columns
// (keys-major rows, up to 128 contiguous bytes each) and transposes it through LDS into
// query rows, written whole.
#include "cm_common.h"
#include "cm_rowops_math.h"

#include <algorithm>

namespace cm {
namespace {

enum : uint32_t { OP_ADD = 0, OP_SUB, OP_MUL, OP_DIV, OP_RELU, OP_RELU6, OP_LEAKY, OP_SILU, OP_GELU,
                  OP_GELU_TANH, OP_SOFTMAX, OP_SOFTMAX_T };
enum : uint32_t { ACT_NONE = 0, ACT_RELU, ACT_RELU6, ACT_LEAKY, ACT_SILU, ACT_GELU, ACT_GELU_TANH };

__device__ __forceinline__ int sat16(int v) { return v > 32767 ? 32767 : (v < -32768 ? -32768 : v); }

// One lane of op 0..9 before the activation (_simulate.py:721-746 on raw lanes).
template <uint32_t OP>
__device__ __forceinline__ int op_lane(int a, int b) {
    if constexpr (OP == OP_ADD) return sat16(a + b);
    else if constexpr (OP == OP_SUB) return sat16(a - b);
    else if constexpr (OP == OP_MUL) return sat16((a * b) >> 8);          // floor: arithmetic shift
    else if constexpr (OP == OP_DIV) {
        if (b == 0) return a > 0 ? 32767 : (a < 0 ? -32768 : 0);
        return sat16((a * 256) / b);                                      // truncates toward zero
    } else if constexpr (OP == OP_RELU) return a < 0 ? 0 : a;
    else if constexpr (OP == OP_RELU6) return a < 0 ? 0 : (a > 1536 ? 1536 : a);
    else return a;                                                        // activation ops
}

// The fused activation (act register or the activation op's own).  LeakyReLU:
// rne(t * alpha[15:0] / 2^16) for t < 0 (exact: |t * alpha| < 2^31).
__device__ __forceinline__ int act_lane(uint32_t act, int t, uint32_t alpha16, const uint8_t* tab,
                                        uint32_t len) {
    switch (act) {
    case ACT_RELU: return t < 0 ? 0 : t;
    case ACT_RELU6: return t < 0 ? 0 : (t > 1536 ? 1536 : t);
    case ACT_LEAKY: {
        if (t >= 0) return t;
        long long p = (long long)t * (long long)alpha16;
        long long q = p >> 16, r = p - (q << 16);
        q += (r > 32768 || (r == 32768 && (q & 1))) ? 1 : 0;
        return (int)q;
    }
    case ACT_SILU: case ACT_GELU: case ACT_GELU_TANH: {
        uint32_t at = (uint32_t)(t < 0 ? -t : t);
        return (t > 0 ? t : 0) - (at < len ? (int)tab[at] : 0);
    }
    default: return t;
    }
}

template <uint32_t OP>
__global__ __launch_bounds__(256) void vectorop_kernel(const int16_t* __restrict__ a,
                                                       const int16_t* __restrict__ b,
                                                       int16_t* __restrict__ c, uint32_t size,
                                                       uint32_t outer, uint64_t a_inc, uint64_t b_inc,
                                                       uint32_t act, uint32_t alpha,
                                                       const uint8_t* __restrict__ act_tab,
                                                       uint32_t act_len) {
    __shared__ __attribute__((aligned(16))) uint8_t tab[kActTabBytes];
    const bool table = act >= ACT_SILU && act <= ACT_GELU_TANH;
    if (table) {                    // 16-byte loads of the table (act_len <= 4096, a 16-byte aligned image)
        for (uint32_t i = threadIdx.x; i < (act_len + 15) / 16; i += blockDim.x)
            reinterpret_cast<int4*>(tab)[i] = reinterpret_cast<const int4*>(act_tab)[i];
        __syncthreads();
    }
    const uint32_t wpr = (size + 7) >> 3;                                  // words per run
    const uint64_t total = (uint64_t)wpr * outer;
    const uint32_t alpha16 = alpha & 0xFFFFu;
    for (uint64_t w = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; w < total;
         w += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t o = w / wpr;
        const uint32_t wi = (uint32_t)(w - o * wpr);
        const uint32_t base = wi * 8;
        int4 av = *reinterpret_cast<const int4*>(a + o * a_inc + base);
        int4 bv = make_int4(0, 0, 0, 0);
        if constexpr (OP < OP_RELU) bv = *reinterpret_cast<const int4*>(b + o * b_inc + base);
        const int16_t* al = reinterpret_cast<const int16_t*>(&av);
        const int16_t* bl = reinterpret_cast<const int16_t*>(&bv);
        int4 cv;
        int16_t* cl = reinterpret_cast<int16_t*>(&cv);
#pragma unroll
        for (int l = 0; l < 8; l++) {
            const bool live = base + l < size;
            int x = live ? al[l] : 0, y = live ? bl[l] : 0;
            int r = act_lane(act, op_lane<OP>(x, y), alpha16, tab, act_len);
            cl[l] = (int16_t)(live ? r : 0);
        }
        store_stream(c + o * (a_inc + b_inc) + base, cv);
    }
}

// vectorop_kernel over `outer` runs of `size` elements (size a multiple of 64) whose outputs
// are the rows of a matmul's A (row o at c + o size), also writing the output's byte planes and
// its row sums per 1024 columns (APlanes; c null: the planes alone): a wavefront per (row, 1024-column slab), two
// 8-element units per lane, the slab's sum by a wavefront reduction.  Few workgroups per
// compute unit (grid-stride) when an activation table is staged.
template <uint32_t OP>
__global__ __launch_bounds__(256) void vectorop_planes_kernel(const int16_t* __restrict__ a,
                                                              const int16_t* __restrict__ b,
                                                              int16_t* __restrict__ c, uint32_t size,
                                                              uint32_t outer, uint64_t a_inc, uint64_t b_inc,
                                                              uint32_t act, uint32_t alpha,
                                                              const uint8_t* __restrict__ act_tab,
                                                              uint32_t act_len, APlanes po) {
    __shared__ __attribute__((aligned(16))) uint8_t tab[kActTabBytes];
    const bool table = act >= ACT_SILU && act <= ACT_GELU_TANH;
    if (table) {
        for (uint32_t i = threadIdx.x; i < (act_len + 15) / 16; i += blockDim.x)
            reinterpret_cast<int4*>(tab)[i] = reinterpret_cast<const int4*>(act_tab)[i];
        __syncthreads();
    }
    const uint32_t lane = threadIdx.x & 63, units = size / 8, nslab = (size + 1023) / 1024;
    const uint32_t alpha16 = alpha & 0xFFFFu;
    const uint64_t tasks = (uint64_t)outer * nslab;
    for (uint64_t t = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6); t < tasks; t += (uint64_t)gridDim.x * 4) {
        const uint64_t o = t / nslab;
        const uint32_t sl = (uint32_t)(t - o * nslab);
        int32_t sum = 0;
#pragma unroll
        for (uint32_t jj = 0; jj < 2; jj++) {
            const uint32_t u = sl * 128 + jj * 64 + lane;
            if (u >= units) continue;
            const uint32_t base = u * 8;
            const int4 av = *reinterpret_cast<const int4*>(a + o * a_inc + base);
            int4 bv = make_int4(0, 0, 0, 0);
            if constexpr (OP < OP_RELU) bv = *reinterpret_cast<const int4*>(b + o * b_inc + base);
            const int16_t* al = reinterpret_cast<const int16_t*>(&av);
            const int16_t* bl = reinterpret_cast<const int16_t*>(&bv);
            int4 cv;
            int16_t* cl = reinterpret_cast<int16_t*>(&cv);
#pragma unroll
            for (int l = 0; l < 8; l++) cl[l] = (int16_t)act_lane(act, op_lane<OP>(al[l], bl[l]), alpha16, tab, act_len);
            if (c != nullptr) store_stream(c + o * (a_inc + b_inc) + base, cv);
            uint2 h, lw;
            split8(cv, h, lw);
            *reinterpret_cast<uint2*>(po.hi + o * po.k + base) = h;
            *reinterpret_cast<uint2*>(po.lo + o * po.k + base) = lw;
            sum += sum8(cv);
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
        if (lane == 0) po.part[(uint64_t)sl * po.lines + o] = sum;
    }
}

// ---------------------------------------------------------------- softmax
// One vector (vectorop_smx.py:50-66): over its first v scores x_j (v = smx_valid),
//   m = max x_j,  d_j = m - x_j,  y_j = (d_j Cm) >> Cs,
//   e_j = TAB[y_j mod 4096] >> (y_j div 4096)     (0 once y_j div 4096 >= 17: TAB <= 2^16),
//   S = sum e_j,  R = floor(2^40 / S),  P_j = min((e_j R + 2^(39 - f_p)) >> (40 - f_p), 32767),
// and P_j = 0 for j >= v.
//
// e depends on d alone and y grows with d, so e(d) = 0 from dlim on, the least d with
// y(d) >= 17 * 4096 (the host computes it).  Where dlim <= kEtabMax every workgroup builds
// e(0 .. dlim) in LDS (e(dlim) = 0) and a pair of scores costs a packed 16-bit subtraction,
// clamp and shift (the byte offsets 4 d fit 16 bits) and two LDS reads; steeper
// exponentials (larger dlim) stage TAB and compute e per element.
//
// P in double: e R 2^(f_p - 40) + 1/2 is exact (below 2^41, at most 41 significant bits), so
// its truncation is the integer formula's floor, and the pack to int16 saturates at 32767
// (v_cvt_pk_i16_i32).  R = floor(2^40 / S) comes from the correctly rounded quotient, less
// one where that rounded up to the next integer.
//
// A row is held by 16 lanes (one DPP row of the wavefront) as 16-byte words: lane l16 holds
// words l16 + 16 k, k < KW.  Max and sum reduce over the 16 lanes in four DPP steps that
// leave the result in every lane; a wavefront works on four rows at once, so the per-row
// arithmetic (the division) is shared by them.
constexpr uint32_t kEtabMax = 16383;          // largest dlim with e(d) tabulated in LDS (4 dlim < 2^16)
constexpr uint32_t kSmxDead = 65536;          // d given to scores past v: e = 0 in both forms

struct SmxRegs {
    uint32_t cm, cs, fp, valid0, period, dlim;
};


__device__ __forceinline__ uint32_t smx_valid(uint32_t q, uint32_t n, const SmxRegs& r) {
    const uint32_t v = r.valid0 + (r.period ? q % r.period : 0u);
    return v < n ? v : n;
}

// Reductions over the 16 lanes of a DPP row; every lane of the row gets the result.
__device__ __forceinline__ int row16_max(int x) {
    x = max(x, __builtin_amdgcn_update_dpp(INT32_MIN, x, 0xB1, 0xF, 0xF, false));    // quad_perm [1,0,3,2]
    x = max(x, __builtin_amdgcn_update_dpp(INT32_MIN, x, 0x4E, 0xF, 0xF, false));    // quad_perm [2,3,0,1]
    x = max(x, __builtin_amdgcn_update_dpp(INT32_MIN, x, 0x141, 0xF, 0xF, false));   // row_half_mirror
    x = max(x, __builtin_amdgcn_update_dpp(INT32_MIN, x, 0x140, 0xF, 0xF, false));   // row_mirror
    return x;
}

__device__ __forceinline__ uint32_t row16_sum(uint32_t x) {
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0xB1, 0xF, 0xF, false);
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x4E, 0xF, 0xF, false);
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x141, 0xF, 0xF, false);
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x140, 0xF, 0xF, false);
    return x;
}

// Sum over aligned groups of N consecutive lanes (N = 4, 8 or 16, within a DPP row); every lane
// of a group gets the group's sum.
template <uint32_t N>
__device__ __forceinline__ int group_sum(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false);          // quad_perm [1,0,3,2]
    x += __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false);          // quad_perm [2,3,0,1]
    if constexpr (N >= 8) x += __builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false);   // row_half_mirror
    if constexpr (N >= 16) x += __builtin_amdgcn_update_dpp(0, x, 0x140, 0xF, 0xF, false);  // row_mirror
    return x;
}

// The same over the whole wavefront (all 64 lanes active), uniform.
__device__ __forceinline__ int wave_max(int x) {
    const int r = row16_max(x);
    return max(max(__builtin_amdgcn_readlane(r, 0), __builtin_amdgcn_readlane(r, 16)),
               max(__builtin_amdgcn_readlane(r, 32), __builtin_amdgcn_readlane(r, 48)));
}

__device__ __forceinline__ uint32_t wave_sum(uint32_t x) {
    const int r = (int)row16_sum(x);
    return (uint32_t)__builtin_amdgcn_readlane(r, 0) + (uint32_t)__builtin_amdgcn_readlane(r, 16) +
           (uint32_t)__builtin_amdgcn_readlane(r, 32) + (uint32_t)__builtin_amdgcn_readlane(r, 48);
}

// LDS words the exponential table takes: e(0 .. dlim), or TAB; a multiple of 4.
__host__ __device__ constexpr uint32_t smx_tab_words(bool etab, uint32_t dlim) {
    return etab ? ((dlim + 1 + 3) & ~3u) : 4096u;
}

// e(d) for d < dlim of one (Cm, Cs), zero from dlim to the table's end (`words` entries):
// the per-(Cm, Cs) table the kernels stage, built once on the device.
__global__ void smx_etab_kernel(uint32_t* __restrict__ out, uint32_t words, const int32_t* __restrict__ gtab,
                                SmxRegs r) {
    for (uint32_t d = blockIdx.x * blockDim.x + threadIdx.x; d < words; d += gridDim.x * blockDim.x) {
        const uint32_t y = (uint32_t)(((uint64_t)d * r.cm) >> r.cs);
        out[d] = d < r.dlim ? (uint32_t)gtab[y & 4095] >> ((y >> 12) & 31) : 0u;   // d < dlim: y < 17 * 4096
    }
}

// A workgroup's exponential table is n4 16-byte words at tsrc (the e(d) table or TAB).  Its
// loads issue first, up to kStageWords per lane into registers, so that they return ahead
// of the loads the kernel issues next; smx_stage_store then writes them to LDS.
constexpr int kStageWords = 4;

struct SmxStage {
    int4 v[kStageWords];
};

__device__ __forceinline__ void smx_stage_load(SmxStage& st, const int4* __restrict__ tsrc, uint32_t n4) {
#pragma unroll
    for (int j = 0; j < kStageWords; j++) {
        const uint32_t i = threadIdx.x + j * blockDim.x;
        st.v[j] = i < n4 ? tsrc[i] : make_int4(0, 0, 0, 0);
    }
}

__device__ __forceinline__ void smx_stage_store(const SmxStage& st, uint32_t* tab, const int4* __restrict__ tsrc,
                                                uint32_t n4) {
    int4* t4 = reinterpret_cast<int4*>(tab);
#pragma unroll
    for (int j = 0; j < kStageWords; j++) {
        const uint32_t i = threadIdx.x + j * blockDim.x;
        if (i < n4) t4[i] = st.v[j];
    }
    for (uint32_t i = threadIdx.x + kStageWords * blockDim.x; i < n4; i += blockDim.x) t4[i] = tsrc[i];
}

// e(d), d <= 65536 (kSmxDead gives 0).
template <bool ETAB>
__device__ __forceinline__ uint32_t smx_e(uint32_t d, const SmxRegs& r, const uint32_t* tab) {
    if constexpr (ETAB) {
        return tab[min(d, r.dlim)];
    } else {
        const uint32_t y = (uint32_t)(((uint64_t)(d & 0x1FFFFu) * (r.cm & 0xFFFFFFu)) >> r.cs);
        const uint32_t t = tab[y & 4095];
        return d < r.dlim ? t >> ((y >> 12) & 31) : 0u;
    }
}

// R 2^(f_p - 40) as a double; S >= 2^16 whenever a score is valid (the maximum's e is
// TAB[0] = 2^16), so R <= 2^24; S = 0 gives 0.
__device__ __forceinline__ double smx_rscale(uint32_t S, const SmxRegs& r) {
    const uint32_t s1 = S ? S : 65536u;
    uint32_t R = (uint32_t)(1099511627776.0 / (double)s1);
    if ((uint64_t)R * s1 > ((uint64_t)1 << 40)) R--;
    return ldexp((double)(S ? R : 0u), (int)r.fp - 40);
}

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// e of the eight scores of one word (element base of the row; those from v on are dead).
template <bool ETAB>
__device__ __forceinline__ void smx_word_e(const int4& xw, int m, uint32_t base, uint32_t v, const SmxRegs& r,
                                           const uint32_t* tab, uint32_t (&e)[8]) {
    if constexpr (ETAB) {
        const uint32_t* xs = reinterpret_cast<const uint32_t*>(&xw);
        const u16x2 m2 = {(unsigned short)m, (unsigned short)m};
        const u16x2 dl2 = {(unsigned short)r.dlim, (unsigned short)r.dlim};
        u16x2 d[4];
#pragma unroll
        for (int p = 0; p < 4; p++) d[p] = m2 - __builtin_bit_cast(u16x2, xs[p]);   // max - x < 2^16
        if (base + 8 > v) {
#pragma unroll
            for (int p = 0; p < 4; p++) {
                if (base + 2 * p >= v) d[p].x = 0xFFFF;                          // clamps to dlim: e = 0
                if (base + 2 * p + 1 >= v) d[p].y = 0xFFFF;
            }
        }
        const char* tb = reinterpret_cast<const char*>(tab);
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const uint32_t ab = __builtin_bit_cast(uint32_t, __builtin_elementwise_min(d[p], dl2) << 2);
            e[2 * p] = *reinterpret_cast<const uint32_t*>(tb + (ab & 0xFFFFu));
            e[2 * p + 1] = *reinterpret_cast<const uint32_t*>(tb + (ab >> 16));
        }
    } else {
        const int16_t* xl = reinterpret_cast<const int16_t*>(&xw);
        uint32_t d[8];
#pragma unroll
        for (int l = 0; l < 8; l++) d[l] = (uint32_t)(m - (int)xl[l]);
        if (base + 8 > v) {
#pragma unroll
            for (int l = 0; l < 8; l++) d[l] = base + l < v ? d[l] : kSmxDead;
        }
#pragma unroll
        for (int l = 0; l < 8; l++) e[l] = smx_e<false>(d[l], r, tab);
    }
}

// Two P lanes packed, saturated to 32767.  e rs + 1/2 < 2^30 + 1 for f_p <= 30; f_p = 31
// (CLAMP) can reach 2^31 and clamps in double before the conversion.
template <bool CLAMP>
__device__ __forceinline__ int smx_p2(uint32_t e0, uint32_t e1, double rs) {
    double t0 = fma((double)e0, rs, 0.5), t1 = fma((double)e1, rs, 0.5);
    if constexpr (CLAMP) {
        t0 = fmin(t0, 32767.0);
        t1 = fmin(t1, 32767.0);
    }
    return __builtin_bit_cast(int, __builtin_amdgcn_cvt_pk_i16((int)t0, (int)t1));
}

template <int KW, bool CLAMP>
__device__ __forceinline__ void smx_store(const uint32_t (&e)[KW][8], double rs, uint32_t words,
                                          int16_t* __restrict__ out, uint32_t l16) {
#pragma unroll
    for (int k = 0; k < KW; k++) {
        const uint32_t w = l16 + 16 * k;
        if (w < words)
            store_stream(out + 8 * w, make_int4(smx_p2<CLAMP>(e[k][0], e[k][1], rs), smx_p2<CLAMP>(e[k][2], e[k][3], rs),
                                                smx_p2<CLAMP>(e[k][4], e[k][5], rs), smx_p2<CLAMP>(e[k][6], e[k][7], rs)));
    }
}

__device__ __forceinline__ int4 smx_pack(const uint32_t (&e)[8], double rs) {
    return make_int4(smx_p2<true>(e[0], e[1], rs), smx_p2<true>(e[2], e[3], rs), smx_p2<true>(e[4], e[5], rs),
                     smx_p2<true>(e[6], e[7], rs));
}

// The softmax of one row held by 16 lanes, written to out as whole words (the lanes past
// v are 0); words = ceil(n / 8) <= 16 KW.
template <int KW, bool ETAB>
__device__ __forceinline__ void smx_row16(const int4 (&xv)[KW], uint32_t words, uint32_t v, const SmxRegs& r,
                                          const uint32_t* tab, int16_t* __restrict__ out, uint32_t l16) {
    int m = -32768;
#pragma unroll
    for (int k = 0; k < KW; k++) {
        const uint32_t base = 8 * (l16 + 16 * k);
        const int16_t* xl = reinterpret_cast<const int16_t*>(&xv[k]);
        if (base + 8 <= v) {
#pragma unroll
            for (int l = 0; l < 8; l++) m = max(m, (int)xl[l]);
        } else {
#pragma unroll
            for (int l = 0; l < 8; l++) m = max(m, base + l < v ? (int)xl[l] : -32768);
        }
    }
    m = row16_max(m);
    uint32_t e[KW][8];
    uint32_t S = 0;
#pragma unroll
    for (int k = 0; k < KW; k++) {
        smx_word_e<ETAB>(xv[k], m, 8 * (l16 + 16 * k), v, r, tab, e[k]);
#pragma unroll
        for (int l = 0; l < 8; l++) S += e[k][l];
    }
    const double rs = smx_rscale(row16_sum(S), r);
    if (r.fp < 31) smx_store<KW, false>(e, rs, words, out, l16);
    else smx_store<KW, true>(e, rs, words, out, l16);
}

// Row mode over `total` rows (row g of matrix g / rows, at a + (g / rows) a_bs + (g mod
// rows) a_inc, its index for the valid count row0 + g mod rows).  Workgroups stay resident
// and take groups of 16 lanes' rows in turn, so the table is staged once per workgroup, its
// loads ahead of the first rows'.  A group steps by the grid's row slots with the matrix /
// row split and both offsets carried, not divided.
template <int KW, bool ETAB>
__global__ __launch_bounds__(1024, KW <= 3 ? 8 : 4) void softmax_rows_kernel(
    const int16_t* __restrict__ a, int16_t* __restrict__ c, uint32_t n, uint32_t rows, uint32_t total, uint32_t row0,
    uint64_t a_inc, uint64_t c_inc, uint64_t a_bs, uint64_t c_bs, SmxRegs r, const int4* __restrict__ tsrc,
    uint32_t tab_n4) {
    extern __shared__ __attribute__((aligned(16))) uint32_t smx_lds[];
    SmxStage stg;
    smx_stage_load(stg, tsrc, tab_n4);
    const uint32_t l16 = threadIdx.x & 15, words = (n + 7) >> 3;
    const uint32_t per_wg = blockDim.x >> 4, slots = gridDim.x * per_wg;
    uint32_t g = blockIdx.x * per_wg + (threadIdx.x >> 4);
    const uint32_t sdiv = slots / rows, smod = slots - sdiv * rows;
    const uint32_t bt = g / rows;
    uint32_t row = g - bt * rows;
    uint64_t oa = bt * a_bs + row * a_inc, oc = bt * c_bs + row * c_inc;
    const uint64_t da = sdiv * a_bs + smod * a_inc, dc = sdiv * c_bs + smod * c_inc;
    const uint64_t wa = a_bs - rows * a_inc, wc = c_bs - rows * c_inc;   // the step into the next matrix (mod 2^64)
    int4 xv[KW];
    auto load_row = [&]() {
#pragma unroll
        for (int k = 0; k < KW; k++) {
            const uint32_t w = l16 + 16 * k;
            xv[k] = w < words ? *reinterpret_cast<const int4*>(a + oa + 8 * w) : make_int4(0, 0, 0, 0);
        }
    };
    // the first rows' loads follow the table's (rows of up to 3 words a lane: longer rows
    // would hold too many registers across the staging)
    constexpr bool kEarly = KW <= 3;
    if (kEarly && g < total) load_row();
    smx_stage_store(stg, smx_lds, tsrc, tab_n4);
    __syncthreads();
    for (bool first = kEarly; g < total; g += slots, first = false) {
        if (!first) load_row();
        smx_row16<KW, ETAB>(xv, words, smx_valid(row0 + row, n, r), r, smx_lds, c + oc, l16);
        row += smod;
        oa += da;
        oc += dc;
        if (row >= rows) {
            row -= rows;
            oa += wa;
            oc += wc;
        }
    }
}

// Rows longer than 16 x 128 words' worth (n > 1024): a wavefront per row, three passes over
// the row (max, sum, output), e recomputed from the table in the last.
template <bool ETAB>
__global__ __launch_bounds__(1024) void softmax_long_kernel(const int16_t* __restrict__ a,
                                                            int16_t* __restrict__ c, uint32_t n, uint32_t rows,
                                                            uint32_t total, uint32_t row0, uint64_t a_inc,
                                                            uint64_t c_inc, uint64_t a_bs, uint64_t c_bs, SmxRegs r,
                                                            const int4* __restrict__ tsrc, uint32_t tab_n4) {
    extern __shared__ __attribute__((aligned(16))) uint32_t smx_lds[];
    SmxStage stg;
    smx_stage_load(stg, tsrc, tab_n4);
    smx_stage_store(stg, smx_lds, tsrc, tab_n4);
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63, words = (n + 7) >> 3;
    const uint32_t slots = gridDim.x * (blockDim.x >> 6);
    for (uint32_t g = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); g < total; g += slots) {
        const uint32_t bt = g / rows, row = g - bt * rows;
        const int16_t* x = a + bt * a_bs + (uint64_t)row * a_inc;
        int16_t* p = c + bt * c_bs + (uint64_t)row * c_inc;
        const uint32_t v = smx_valid(row0 + row, n, r);
        int m = -32768;
        for (uint32_t w = lane; w < words; w += 64) {
            const int4 xv = *reinterpret_cast<const int4*>(x + 8 * w);
            const int16_t* xl = reinterpret_cast<const int16_t*>(&xv);
#pragma unroll
            for (int l = 0; l < 8; l++) m = max(m, 8 * w + l < v ? (int)xl[l] : -32768);
        }
        m = wave_max(m);
        uint32_t S = 0;
        for (uint32_t w = lane; w < words; w += 64) {
            const int4 xv = *reinterpret_cast<const int4*>(x + 8 * w);
            const int16_t* xl = reinterpret_cast<const int16_t*>(&xv);
#pragma unroll
            for (int l = 0; l < 8; l++)
                S += smx_e<ETAB>(8 * w + l < v ? (uint32_t)(m - (int)xl[l]) : kSmxDead, r, smx_lds);
        }
        const double rs = smx_rscale(wave_sum(S), r);
        for (uint32_t w = lane; w < words; w += 64) {
            const int4 xv = *reinterpret_cast<const int4*>(x + 8 * w);
            const int16_t* xl = reinterpret_cast<const int16_t*>(&xv);
            uint32_t e[8];
#pragma unroll
            for (int l = 0; l < 8; l++)
                e[l] = smx_e<ETAB>(8 * w + l < v ? (uint32_t)(m - (int)xl[l]) : kSmxDead, r, smx_lds);
            store_stream(p + 8 * w, smx_pack(e, rs));
        }
    }
}

// Column mode: s[keys][queries] (row stride a_inc) -> P[q][keys] at c + q c_inc, for
// `batch` matrices at a + h a_bs, c + h c_bs.  A workgroup of 16 qt lanes takes qt query
// columns (qt = 16, 32, 48 or 64) of one matrix: the [n keys][qt] block is read 2 qt
// contiguous bytes per key row and written transposed into LDS as qt query rows (pitch
// n + 8 keys, so the transposing writes spread over the banks); each 16 lanes then take
// one query row through the row computation.  Tiles are numbered so that the workgroups of
// one XCD (workgroup id mod 8) take neighbouring tiles, whose key rows share cache lines.
constexpr uint32_t kColsMaxKeys = 1024;

__host__ __device__ constexpr uint32_t cols_pitch(uint32_t n) { return ((n + 7) & ~7u) + 8; }

template <int KW, bool ETAB>
__global__ __launch_bounds__(1024, KW <= 3 ? 8 : 4) void softmax_cols_kernel(const int16_t* __restrict__ s,
                                                            int16_t* __restrict__ c, uint32_t n, uint32_t nq,
                                                            uint32_t qt, uint32_t tiles_q, uint32_t tiles,
                                                            uint64_t a_inc, uint64_t c_inc, uint64_t a_bs,
                                                            uint64_t c_bs, SmxRegs r,
                                                            const int4* __restrict__ tsrc, uint32_t tab_n4) {
    extern __shared__ __attribute__((aligned(16))) uint32_t smx_lds[];
    const uint32_t per_xcd = (tiles + 7) >> 3;
    const uint32_t tile = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (tile >= tiles) return;                           // whole workgroup: before any barrier
    const uint32_t h = tile / tiles_q, q0 = (tile - h * tiles_q) * qt;
    const uint32_t t = threadIdx.x, nt = blockDim.x;
    const uint32_t pitch = cols_pitch(n), words = (n + 7) >> 3;
    int16_t* blk = reinterpret_cast<int16_t*>(smx_lds + tab_n4 * 4);   // [qt][pitch]
    const int16_t* sh = s + h * a_bs;
    SmxStage stg;
    smx_stage_load(stg, tsrc, tab_n4);
    if ((a_inc & 7) == 0) {
        // 8 queries (16 bytes) of key row j per lane, written transposed: blk[q][j].  The
        // qt / 8 chunks of a key row go to consecutive lanes and a workgroup (16 qt lanes)
        // covers 128 key rows a step, so n <= 1024 keys take at most 8 loads per lane, all
        // issued before the first write.
        const uint32_t chunks = qt >> 3, ch = t % chunks, j0 = t / chunks, q = q0 + 8 * ch;
        int4 bv[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const uint32_t j = j0 + 128 * u;
            bv[u] = (j < n && q < nq) ? *reinterpret_cast<const int4*>(sh + j * a_inc + q) : make_int4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const uint32_t j = j0 + 128 * u;
            const int16_t* vl = reinterpret_cast<const int16_t*>(&bv[u]);
            if (j < n) {
#pragma unroll
                for (int l = 0; l < 8; l++) blk[(8 * ch + l) * pitch + j] = vl[l];
            }
        }
    } else {
        for (uint32_t i = t; i < n * qt; i += nt) {
            const uint32_t j = i / qt, qq = i - j * qt;
            blk[qq * pitch + j] = q0 + qq < nq ? sh[j * a_inc + q0 + qq] : (int16_t)0;
        }
    }
    // keys n .. pitch of every row are zero (their P lanes are written as 0)
    const uint32_t pad = pitch - n;
    for (uint32_t i = t; i < qt * pad; i += nt) blk[(i / pad) * pitch + n + i % pad] = 0;
    smx_stage_store(stg, smx_lds, tsrc, tab_n4);
    __syncthreads();
    const uint32_t l16 = t & 15;
    for (uint32_t qq = t >> 4; qq < qt; qq += nt >> 4) {
        const uint32_t q = q0 + qq;
        if (q >= nq) break;
        const int16_t* row = blk + qq * pitch;
        int4 xv[KW];
#pragma unroll
        for (int k = 0; k < KW; k++) {
            const uint32_t w = l16 + 16 * k;
            xv[k] = w < words ? *reinterpret_cast<const int4*>(row + 8 * w) : make_int4(0, 0, 0, 0);
        }
        smx_row16<KW, ETAB>(xv, words, smx_valid(q, n, r), r, smx_lds, c + h * c_bs + (uint64_t)q * c_inc, l16);
    }
}

// Words per lane of the 16-lane row form for a row of `words` words (0: beyond it).
uint32_t smx_kw(uint32_t words) {
    for (uint32_t kw : {1u, 2u, 3u, 4u, 6u, 8u})
        if (words <= 16 * kw) return kw;
    return 0;
}

// Workgroups of `kernel` one compute unit holds at `block` lanes and `lds` bytes (1 if the
// runtime does not say).
int blocks_per_cu(const void* kernel, int block, size_t lds) {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kernel, block, lds) != hipSuccess) {
        (void)hipGetLastError();
        nb = 1;
    }
    return nb > 0 ? nb : 1;
}

using SmxRowsFn = void (*)(const int16_t*, int16_t*, uint32_t, uint32_t, uint32_t, uint32_t, uint64_t, uint64_t,
                           uint64_t, uint64_t, SmxRegs, const int4*, uint32_t);
using SmxColsFn = void (*)(const int16_t*, int16_t*, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint64_t,
                           uint64_t, uint64_t, uint64_t, SmxRegs, const int4*, uint32_t);

// The workgroups' table: e(d) for this (Cm, Cs) from the device's cache, built on `s` by the
// first call that needs it (later calls on other streams wait for that build until it is
// seen complete); nullptr when the cache is full (the caller then stages TAB).
constexpr size_t kEtabCacheEntries = 1024;

int smx_etab(DeviceState* st, const SmxRegs& r, hipStream_t s, const uint32_t** out) {
    std::lock_guard<std::mutex> lk(st->smx_mu);
    *out = nullptr;
    for (SmxEtab& e : st->smx_etabs) {
        if (e.cm != r.cm || e.cs != r.cs) continue;
        if (!e.done) {
            const hipError_t q = hipEventQuery(e.ready);
            if (q == hipSuccess) {
                e.done = true;
            } else if (q == hipErrorNotReady) {
                (void)hipGetLastError();
                CM_HIP_CHECK(hipStreamWaitEvent(s, e.ready, 0));
            } else {
                return hip_fail(q, "hipEventQuery (softmax table)");
            }
        }
        *out = e.table;
        return CM_OK;
    }
    if (st->smx_etabs.size() >= kEtabCacheEntries) return CM_OK;
    SmxEtab e;
    e.cm = r.cm;
    e.cs = r.cs;
    const uint32_t words = smx_tab_words(true, r.dlim);
    CM_HIP_CHECK(hipMalloc(&e.table, (size_t)words * 4));
    CM_HIP_CHECK(hipEventCreateWithFlags(&e.ready, hipEventDisableTiming));
    CM_LAUNCH("smx_etab_kernel", smx_etab_kernel, dim3(ceil_div(words, 256)), dim3(256), 0, s, e.table, words,
              st->smx_tab, r);
    CM_HIP_CHECK(hipEventRecord(e.ready, s));
    st->smx_etabs.push_back(e);
    *out = e.table;
    return CM_OK;
}

template <bool ETAB>
SmxRowsFn rows_kernel(uint32_t kw) {
    switch (kw) {
    case 1: return softmax_rows_kernel<1, ETAB>;
    case 2: return softmax_rows_kernel<2, ETAB>;
    case 3: return softmax_rows_kernel<3, ETAB>;
    case 4: return softmax_rows_kernel<4, ETAB>;
    case 6: return softmax_rows_kernel<6, ETAB>;
    case 8: return softmax_rows_kernel<8, ETAB>;
    default: return softmax_long_kernel<ETAB>;
    }
}

template <bool ETAB>
SmxColsFn cols_kernel(uint32_t kw) {
    switch (kw) {
    case 1: return softmax_cols_kernel<1, ETAB>;
    case 2: return softmax_cols_kernel<2, ETAB>;
    case 3: return softmax_cols_kernel<3, ETAB>;
    case 4: return softmax_cols_kernel<4, ETAB>;
    case 6: return softmax_cols_kernel<6, ETAB>;
    default: return softmax_cols_kernel<8, ETAB>;
    }
}

template <bool ETAB>
int launch_rows(const int16_t* a, int16_t* c, uint32_t n, uint32_t rows, uint32_t total, uint32_t row0,
                uint64_t a_inc, uint64_t c_inc, uint64_t a_bs, uint64_t c_bs, const SmxRegs& r, const int4* tsrc,
                const DeviceState* st, hipStream_t s) {
    const uint32_t tab_n4 = smx_tab_words(ETAB, r.dlim) / 4;
    const size_t lds = (size_t)tab_n4 * 16;
    const uint32_t kw = smx_kw((n + 7) >> 3);
    const SmxRowsFn k = rows_kernel<ETAB>(kw);
    // 16 lanes a row: 64 rows per 1024-thread workgroup pass; fewer rows than that per compute
    // unit take smaller workgroups (down to 4 rows), so that they spread over the units
    uint32_t threads = 1024;
    if (kw && ceil_div(total, 64) < st->cus)
        threads = std::min<uint32_t>(1024, std::max<uint32_t>(64, (uint32_t)round_up(16 * ceil_div(total, st->cus), 64)));
    const uint32_t per_wg = kw ? threads / 16 : 16;                   // rows per workgroup pass
    const uint64_t resident = (uint64_t)st->cus * blocks_per_cu(reinterpret_cast<const void*>(k), threads, lds);
    const unsigned blocks = (unsigned)std::min<uint64_t>(ceil_div(total, per_wg), resident);
    if (kw) {
        CM_LAUNCH("softmax_rows_kernel", k, dim3(blocks), dim3(threads), lds, s, a, c, n, rows, total, row0, a_inc,
                  c_inc, a_bs, c_bs, r, tsrc, tab_n4);
    } else {
        CM_LAUNCH("softmax_long_kernel", k, dim3(blocks), dim3(1024), lds, s, a, c, n, rows, total, row0, a_inc, c_inc,
                  a_bs, c_bs, r, tsrc, tab_n4);
    }
    return CM_OK;
}

template <bool ETAB>
int launch_cols(const int16_t* a, int16_t* c, uint32_t n, uint32_t nq, uint32_t batch, uint64_t a_inc,
                uint64_t c_inc, uint64_t a_bs, uint64_t c_bs, const SmxRegs& r, const int4* tsrc,
                const DeviceState* st, hipStream_t s) {
    // queries per tile: the fewest rounds of resident workgroups times the tile height, ties
    // to the wider tile (longer contiguous key-row reads)
    const uint32_t tab_n4 = smx_tab_words(ETAB, r.dlim) / 4;
    const size_t tab = (size_t)tab_n4 * 16;
    const SmxColsFn k = cols_kernel<ETAB>(smx_kw((n + 7) >> 3));
    uint32_t qt = 0;
    uint64_t best = ~0ull;
    for (uint32_t cand : {64u, 48u, 32u}) {
        const size_t lds = tab + (size_t)cand * cols_pitch(n) * sizeof(int16_t);
        if (lds > st->lds_per_block) continue;
        const uint64_t per_cu = blocks_per_cu(reinterpret_cast<const void*>(k), 16 * cand, lds);
        const uint64_t tiles = (uint64_t)batch * ceil_div(nq, cand);
        const uint64_t cost = ceil_div(tiles, (uint64_t)st->cus * per_cu) * cand;
        if (cost < best) {
            best = cost;
            qt = cand;
        }
    }
    if (!qt) qt = 16;                                    // always fits: 16 x 1032 x 2 B + 64 KiB
    const uint32_t tiles_q = ceil_div(nq, qt);
    const uint64_t tiles = (uint64_t)tiles_q * batch;
    if (tiles > 0x7FFFFFF8ull) return fail(CM_EINVAL, "softmax columns: %llu tiles", (unsigned long long)tiles);
    const unsigned grid = (unsigned)((tiles + 7) & ~7ull);
    const size_t lds = tab + (size_t)qt * cols_pitch(n) * sizeof(int16_t);
    if (lds > st->lds_per_block) return fail(CM_EINVAL, "softmax columns: %u keys do not fit the LDS", n);
    CM_LAUNCH("softmax_cols_kernel", k, dim3(grid), dim3(16 * qt), lds, s, a, c, n, nq, qt, tiles_q,
              (uint32_t)tiles, a_inc, c_inc, a_bs, c_bs, r, tsrc, tab_n4);
    return CM_OK;
}

// The softmax unit over `batch` matrices: op 10 rows [outer][size] (row strides a_inc, c_inc),
// op 11 keys-major s[size][outer] -> P[outer][size]; matrix i at a + i a_bs, c + i c_bs.
int launch_softmax(const int16_t* a, int16_t* c, uint32_t size, uint32_t op, uint32_t outer, uint32_t a_inc,
                   uint32_t c_inc, uint32_t smx_cm, uint32_t smx_cfg, uint32_t smx_mask, uint32_t batch,
                   uint64_t a_bs, uint64_t c_bs, DeviceState* st, hipStream_t s) {
    SmxRegs r{smx_cm & 0xFFFFFFu, smx_cfg & 63u, (smx_cfg >> 8) & 31u, smx_mask & 0xFFFFu, smx_mask >> 16, 0};
    r.dlim = smx_dlim(r.cm, r.cs);
    if (size > 65535) return fail(CM_EINVAL, "softmax: %u elements per vector", size);
    if (c_inc & 7) return fail(CM_EALIGN, "softmax: output stride %u not a multiple of 8", c_inc);
    if (!aligned16(a) || !aligned16(c)) return fail(CM_EALIGN, "softmax: a and c must be 16-byte aligned");
    if (batch > 1 && ((a_bs & 7) || (c_bs & 7)))
        return fail(CM_EALIGN, "softmax: batch strides must be multiples of 8 elements");
    if (op == OP_SOFTMAX_T && (outer & ~15u) == 0) return CM_OK;
    if (op == OP_SOFTMAX_T && size > kColsMaxKeys)
        return fail(CM_EINVAL, "softmax columns: %u keys above %u", size, kColsMaxKeys);
    const uint32_t* etab_src = nullptr;
    if (r.dlim <= kEtabMax) {
        const int rc = smx_etab(st, r, s, &etab_src);
        if (rc) return rc;
    }
    const bool etab = etab_src != nullptr;
    const int4* tsrc = reinterpret_cast<const int4*>(etab ? etab_src : reinterpret_cast<const uint32_t*>(st->smx_tab));
    if (op == OP_SOFTMAX) {
        if (a_inc & 7) return fail(CM_EALIGN, "softmax rows: input stride %u not a multiple of 8", a_inc);
        // launches of at most 2^30 rows: whole matrices, or row ranges of one matrix
        constexpr uint64_t kMaxRows = (uint64_t)1 << 30;
        for (uint64_t b0 = 0; b0 < batch;) {
            const uint64_t nb = outer >= kMaxRows ? 1 : std::min<uint64_t>(batch - b0, kMaxRows / outer);
            for (uint64_t r0 = 0; r0 < outer; r0 += kMaxRows) {
                const uint32_t nr = (uint32_t)std::min<uint64_t>(outer - r0, kMaxRows);
                const int16_t* ab = a + b0 * a_bs + r0 * a_inc;
                int16_t* cb = c + b0 * c_bs + r0 * c_inc;
                const uint32_t total = (uint32_t)(nr * nb);
                const int rc = etab ? launch_rows<true>(ab, cb, size, nr, total, (uint32_t)r0, a_inc, c_inc, a_bs,
                                                        c_bs, r, tsrc, st, s)
                                    : launch_rows<false>(ab, cb, size, nr, total, (uint32_t)r0, a_inc, c_inc, a_bs,
                                                         c_bs, r, tsrc, st, s);
                if (rc) return rc;
            }
            b0 += nb;
        }
        return CM_OK;
    }
    const uint32_t nq = outer & ~15u;
    return etab ? launch_cols<true>(a, c, size, nq, batch, a_inc, c_inc, a_bs, c_bs, r, tsrc, st, s)
                : launch_cols<false>(a, c, size, nq, batch, a_inc, c_inc, a_bs, c_bs, r, tsrc, st, s);
}

// ---------------------------------------------------------------- decode attention
// One decode step's attention for a KV group (b, g) in one workgroup: the group's G query
// rows against its cache of C rows, the chain of the unfused nodes
//   s[i][j] = sat16(wrap32(sum_d q[i][d] K[j][d]) >> 8)        (q.K^T, MatmulKernel's wrap rule)
//   P[i][.] = the softmax unit's row mode over s[i][.] (valid keys from the mask register)
//   o[i][d] = sat16(wrap32(sum_j P[i][j] V[j][d]) >> 8)        (P.V)
// without materializing s or P in HBM.  Phase 1: lane l reads word l % W4 of a key row (a
// wavefront's loads cover whole rows), dots its 8 d with every query (v_dot2) and the W4 lanes
// of a row sum by DPP; phase 2: the max and the sum of every query over the workgroup
// (wavefront reductions, then LDS), e from the staged TAB and P by the rule of smx_row16
// (scores past the valid count 0); phase 3: the consecutive lanes of a chunk of 8 d take pairs
// of keys (v_dot2 over the pair) and sum by DPP, then over the wavefronts.  G is a template
// argument, so every loop over the queries unrolls into independent chains.  Head dim HD (32
// or 64): q rows of group bg at q + bg G HD, the caches' rows at kc / vc + bg C HD, o like q.
constexpr uint32_t kDaThreads = 1024;          // four wavefronts a SIMD hide each other's latencies
constexpr uint32_t kDaWaves = kDaThreads / 64;
constexpr uint32_t kDaMaxG = 8;

// The decode step's attention prep of the group, done by its attention workgroup first (the
// decode_prep launch of the row-ops unit, one group's share, the same element rule): q's G
// heads RoPE'd at the position into qr and into the workgroup's query staging, k's head
// RoPE'd into the K cache row at pos, v's head copied into the V cache row; q / k / v rows of
// sequence b at q + b H HD, k / v + b KV HD; the ROPE jobs' parameter blocks (per column of
// those rows, or one entry) and the position's table row (cos [HD], sin [HD]).
struct DaPrep {
    const int16_t *q, *k, *v;
    int16_t *qr, *kc, *vc;
    const int32_t* tab;
    const uint8_t *pq, *pk;
    uint32_t bcq, bck, KV, pos;
};

template <uint32_t HD, uint32_t G, bool PREP>
__global__ __launch_bounds__(kDaThreads) void decode_attn_kernel(const int16_t* __restrict__ q,
                                                                 const int16_t* __restrict__ kc,
                                                                 const int16_t* __restrict__ vc,
                                                                 int16_t* __restrict__ o, uint32_t C, SmxRegs r,
                                                                 const int4* __restrict__ tsrc, DaPrep pp) {
    constexpr uint32_t W4 = HD / 8;                         // 16-byte words of a row
    constexpr uint32_t KPW = 64 / W4;                       // rows a wavefront load covers
    extern __shared__ __attribute__((aligned(16))) uint32_t da_lds[];
    uint32_t* tab = da_lds;                                 // TAB: 4096 words
    uint32_t* qs = tab + 4096;                              // [G][HD / 2] d pairs
    int32_t* red = reinterpret_cast<int32_t*>(qs + kDaMaxG * 32);       // [2][waves][8] reductions
    uint32_t* oacc = reinterpret_cast<uint32_t*>(red + 2 * kDaWaves * kDaMaxG);   // [G][HD] sums of P V
    int16_t* ps = reinterpret_cast<int16_t*>(oacc + kDaMaxG * 64);     // s, then P: [G][C]
    const uint32_t bg = blockIdx.x, t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int16_t* qg = q + (uint64_t)bg * G * HD;
    const int16_t* kg = kc + (uint64_t)bg * C * HD;
    const int16_t* vg = vc + (uint64_t)bg * C * HD;
    typedef short v2s __attribute__((ext_vector_type(2)));

    // ---- phase 1 loads first: KCH rounds of KR rows (one word a lane) in flight
    constexpr uint32_t KR = kDaWaves * KPW, KCH = 8;
    const uint32_t kw = t % W4, krow = t / W4;
    int4 kv[KCH];
    auto load_k = [&](uint32_t j0, uint32_t skip) {      // row `skip` is not read
#pragma unroll
        for (uint32_t u = 0; u < KCH; u++) {
            const uint32_t j = j0 + u * KR + krow;
            kv[u] = j < C && j != skip ? reinterpret_cast<const int4*>(kg + (uint64_t)j * HD)[kw] : make_int4(0, 0, 0, 0);
        }
    };
    SmxStage stg;
    smx_stage_load(stg, tsrc, 1024);                        // ahead of the K loads: staged first
    load_k(0, PREP ? pp.pos : 0xFFFFFFFFu);
    if constexpr (PREP) {
        // the prep, under the loads above: a thread per 8-element word: the group's q words, then k's, then v's
        const uint32_t b = bg / pp.KV, g = bg - b * pp.KV, H = pp.KV * G;
        constexpr uint32_t QW = G * HD / 8, KW = HD / 8;
        for (uint32_t w = t; w < QW + 2 * KW; w += kDaThreads) {
            uint32_t out[4] = {0, 0, 0, 0};
            if (w < QW + KW) {
                const bool isq = w < QW;
                const uint32_t col0 = isq ? g * G * HD + 8 * w : g * HD + 8 * (w - QW);
                const int16_t* row = isq ? pp.q + (uint64_t)b * H * HD : pp.k + (uint64_t)b * pp.KV * HD;
                const uint8_t* prm = isq ? pp.pq : pp.pk;
                const bool bc = (isq ? pp.bcq : pp.bck) != 0;
                const uint32_t d0 = col0 % HD;
                const int4 xw = *reinterpret_cast<const int4*>(row + col0);
                const int4 pw = *reinterpret_cast<const int4*>(row + (d0 < HD / 2 ? col0 + HD / 2 : col0 - HD / 2));
                const uint4 ow = ro::rope_unit8(xw, pw, pp.tab, HD, d0, [&](uint32_t l) { return ro::ld_param(prm, col0 + l, bc); });
                out[0] = ow.x; out[1] = ow.y; out[2] = ow.z; out[3] = ow.w;
                if (isq) {
                    *reinterpret_cast<uint4*>(pp.qr + (uint64_t)b * H * HD + col0) = make_uint4(out[0], out[1], out[2], out[3]);
#pragma unroll
                    for (int e = 0; e < 4; e++) qs[4 * w + e] = out[e];
                } else {
                    *reinterpret_cast<uint4*>(pp.kc + ((uint64_t)bg * C + pp.pos) * HD + 8 * (w - QW)) =
                        make_uint4(out[0], out[1], out[2], out[3]);
                }
            } else {
                const uint32_t c0 = 8 * (w - QW - KW);
                const uint4 x = *reinterpret_cast<const uint4*>(pp.v + (uint64_t)b * pp.KV * HD + g * HD + c0);
                *reinterpret_cast<uint4*>(pp.vc + ((uint64_t)bg * C + pp.pos) * HD + c0) = x;
            }
        }
    }
    if constexpr (!PREP)
        for (uint32_t e = t; e < G * HD / 2; e += kDaThreads) qs[e] = reinterpret_cast<const uint32_t*>(qg)[e];
    for (uint32_t e = t; e < G * HD; e += kDaThreads) oacc[e] = 0u;
    smx_stage_store(stg, tab, tsrc, 1024);
    // orders qs and the prep's cache rows (workgroup-scope release / acquire) before their reads;
    // without the prep only LDS is shared, and the K loads stay in flight
    if constexpr (PREP) __syncthreads();
    else lds_barrier();
    if constexpr (PREP) {
        // the first K loads went out before the prep wrote row pos and left it out: that row now
#pragma unroll
        for (uint32_t u = 0; u < KCH; u++)
            if (u * KR + krow == pp.pos) kv[u] = reinterpret_cast<const int4*>(kg + (uint64_t)pp.pos * HD)[kw];
    }
    uint32_t qv[G][4];                                      // this lane's 8 d of every query
#pragma unroll
    for (uint32_t i = 0; i < G; i++)
#pragma unroll
        for (int w = 0; w < 4; w++) qv[i][w] = qs[i * (HD / 2) + 4 * kw + w];
    for (uint32_t j0 = 0; j0 < C; j0 += KR * KCH) {
        if (j0) load_k(j0, 0xFFFFFFFFu);
#pragma unroll
        for (uint32_t u = 0; u < KCH; u++) {
            int acc[G];
#pragma unroll
            for (uint32_t i = 0; i < G; i++) {
                acc[i] = __builtin_amdgcn_sdot2(__builtin_bit_cast(v2s, qv[i][0]), __builtin_bit_cast(v2s, kv[u].x), 0, false);
                acc[i] = __builtin_amdgcn_sdot2(__builtin_bit_cast(v2s, qv[i][1]), __builtin_bit_cast(v2s, kv[u].y), acc[i], false);
                acc[i] = __builtin_amdgcn_sdot2(__builtin_bit_cast(v2s, qv[i][2]), __builtin_bit_cast(v2s, kv[u].z), acc[i], false);
                acc[i] = __builtin_amdgcn_sdot2(__builtin_bit_cast(v2s, qv[i][3]), __builtin_bit_cast(v2s, kv[u].w), acc[i], false);
                acc[i] = group_sum<W4>(acc[i]);
            }
            const uint32_t j = j0 + u * KR + krow;
            if (kw == 0 && j < C) {
#pragma unroll
                for (uint32_t i = 0; i < G; i++) ps[i * C + j] = (int16_t)min(max(acc[i] >> 8, -32768), 32767);
            }
        }
    }
    // phase 3's lanes: the KPW consecutive lanes of d chunk dc take key pairs kp0 = wave KPW +
    // slot; their first VCH pairs are loaded now, in flight across the softmax
    constexpr uint32_t KPG = kDaThreads / W4, VCH = 4;
    const uint32_t dc = lane / KPW, kp0 = wave * KPW + lane % KPW;
    int4 va[VCH], vb[VCH];
    auto load_v = [&](uint32_t j0) {
#pragma unroll
        for (uint32_t u = 0; u < VCH; u++) {
            const uint32_t j = j0 + u * 2 * KPG;
            va[u] = j < C ? *reinterpret_cast<const int4*>(vg + (uint64_t)j * HD + 8 * dc) : make_int4(0, 0, 0, 0);
            vb[u] = j < C ? *reinterpret_cast<const int4*>(vg + (uint64_t)(j + 1) * HD + 8 * dc) : make_int4(0, 0, 0, 0);
        }
    };
    load_v(2 * kp0);
    lds_barrier();

    // ---- phase 2: the softmax of every query row over its valid keys
    uint32_t v[G];
    int m[G];
#pragma unroll
    for (uint32_t i = 0; i < G; i++) {
        v[i] = smx_valid(bg * G + i, C, r);
        m[i] = -32768;
    }
    for (uint32_t j = t; j < C; j += kDaThreads) {
#pragma unroll
        for (uint32_t i = 0; i < G; i++) m[i] = max(m[i], j < v[i] ? (int)ps[i * C + j] : -32768);
    }
#pragma unroll
    for (uint32_t i = 0; i < G; i++) {
        m[i] = wave_max(m[i]);
        if (lane == 0) red[wave * kDaMaxG + i] = m[i];
    }
    lds_barrier();
#pragma unroll
    for (uint32_t i = 0; i < G; i++) {
        int x = red[i];
#pragma unroll
        for (uint32_t w = 1; w < kDaWaves; w++) x = max(x, red[w * kDaMaxG + i]);
        m[i] = x;
    }
    uint32_t S[G];
#pragma unroll
    for (uint32_t i = 0; i < G; i++) S[i] = 0;
    for (uint32_t j = t; j < C; j += kDaThreads) {
#pragma unroll
        for (uint32_t i = 0; i < G; i++)
            S[i] += j < v[i] ? smx_e<false>((uint32_t)(m[i] - (int)ps[i * C + j]), r, tab) : 0u;
    }
    int32_t* red2 = red + kDaWaves * kDaMaxG;
#pragma unroll
    for (uint32_t i = 0; i < G; i++) {
        S[i] = wave_sum(S[i]);
        if (lane == 0) red2[wave * kDaMaxG + i] = (int32_t)S[i];
    }
    lds_barrier();
    double rs[G];
#pragma unroll
    for (uint32_t i = 0; i < G; i++) {
        uint32_t x = 0;
#pragma unroll
        for (uint32_t w = 0; w < kDaWaves; w++) x += (uint32_t)red2[w * kDaMaxG + i];
        rs[i] = smx_rscale(x, r);
    }
    // P in pairs of keys (C even): a thread reads the scores of its own pairs and overwrites
    // them with P; the barrier above ended every other read of the scores
    for (uint32_t j = 2 * t; j < C; j += 2 * kDaThreads) {
#pragma unroll
        for (uint32_t i = 0; i < G; i++) {
            const uint32_t e0 = j < v[i] ? smx_e<false>((uint32_t)(m[i] - (int)ps[i * C + j]), r, tab) : 0u;
            const uint32_t e1 = j + 1 < v[i] ? smx_e<false>((uint32_t)(m[i] - (int)ps[i * C + j + 1]), r, tab) : 0u;
            *reinterpret_cast<int*>(&ps[i * C + j]) = smx_p2<true>(e0, e1, rs[i]);
        }
    }
    lds_barrier();

    // ---- phase 3: o = P . V, VCH key pairs of a lane in flight at a time
    int acc[G][8];
#pragma unroll
    for (uint32_t i = 0; i < G; i++)
#pragma unroll
        for (int l = 0; l < 8; l++) acc[i][l] = 0;
    for (uint32_t j0 = 2 * kp0; j0 < C; j0 += 2 * KPG * VCH) {
        if (j0 != 2 * kp0) load_v(j0);
#pragma unroll
        for (uint32_t u = 0; u < VCH; u++) {
            const uint32_t j = j0 + u * 2 * KPG;
            if (j >= C) break;
            const uint32_t wa[4] = {(uint32_t)va[u].x, (uint32_t)va[u].y, (uint32_t)va[u].z, (uint32_t)va[u].w};
            const uint32_t wb[4] = {(uint32_t)vb[u].x, (uint32_t)vb[u].y, (uint32_t)vb[u].z, (uint32_t)vb[u].w};
            uint32_t pr[8];                                 // (V[j][d], V[j + 1][d]) for the chunk's 8 d
#pragma unroll
            for (int w = 0; w < 4; w++) {
                pr[2 * w] = __builtin_amdgcn_perm(wb[w], wa[w], 0x05040100u);
                pr[2 * w + 1] = __builtin_amdgcn_perm(wb[w], wa[w], 0x07060302u);
            }
#pragma unroll
            for (uint32_t i = 0; i < G; i++) {
                const uint32_t pp = *reinterpret_cast<const uint32_t*>(&ps[i * C + j]);
#pragma unroll
                for (int l = 0; l < 8; l++)
                    acc[i][l] = __builtin_amdgcn_sdot2(__builtin_bit_cast(v2s, pp), __builtin_bit_cast(v2s, pr[l]),
                                                       acc[i][l], false);
            }
        }
    }
    // sum over the key-pair slots of a wavefront (a DPP group of KPW lanes), then over the
    // wavefronts (LDS atomics: the sums wrap)
#pragma unroll
    for (uint32_t i = 0; i < G; i++)
#pragma unroll
        for (int l = 0; l < 8; l++) {
            const int x = group_sum<KPW>(acc[i][l]);
            if (lane % KPW == 0) atomicAdd(&oacc[i * HD + 8 * dc + l], (uint32_t)x);
        }
    lds_barrier();
    for (uint32_t e = t; e < G * HD; e += kDaThreads)
        o[(uint64_t)bg * G * HD + e] = (int16_t)min(max((int32_t)oacc[e] >> 8, -32768), 32767);
}

typedef void (*DecodeAttnFn)(const int16_t*, const int16_t*, const int16_t*, int16_t*, uint32_t, SmxRegs,
                             const int4*, DaPrep);

template <uint32_t HD, bool PREP = false>
DecodeAttnFn decode_attn_fn(uint32_t g) {
    switch (g) {
    case 1: return decode_attn_kernel<HD, 1, PREP>;
    case 2: return decode_attn_kernel<HD, 2, PREP>;
    case 3: return decode_attn_kernel<HD, 3, PREP>;
    case 4: return decode_attn_kernel<HD, 4, PREP>;
    case 5: return decode_attn_kernel<HD, 5, PREP>;
    case 6: return decode_attn_kernel<HD, 6, PREP>;
    case 7: return decode_attn_kernel<HD, 7, PREP>;
    default: return decode_attn_kernel<HD, 8, PREP>;
    }
}

template <uint32_t OP>
int launch_ew(const int16_t* a, const int16_t* b, int16_t* c, uint32_t size, uint32_t outer,
              uint32_t a_inc, uint32_t b_inc, uint32_t act, uint32_t alpha, DeviceState* st,
              hipStream_t s, void* planes = nullptr) {
    const uint64_t words = (uint64_t)((size + 7) >> 3) * outer;
    const unsigned threads = 256;
    uint64_t blocks = (words + threads - 1) / threads;
    if (planes != nullptr) blocks = ((uint64_t)outer * ((size + 1023) / 1024) + 3) / 4;   // a wavefront per slab
    if (blocks > 65536ull * 8) blocks = 65536ull * 8;
    const uint8_t* tab = st->act_tab;
    uint32_t len = 0;
    if (act >= ACT_SILU && act <= ACT_GELU_TANH) {
        tab = st->act_tab + (act - ACT_SILU) * kActTabBytes;
        len = st->act_len[act - ACT_SILU];
        // every workgroup stages the table: eight per compute unit, each over several words or
        // slabs (measured at 3072 x 3072 ADD + GELU: 9.7 / 10.1 us plain / with planes at eight,
        // 10.2 / 11.9 at four)
        blocks = std::min<uint64_t>(blocks, (uint64_t)st->cus * 8);
    }
    if (planes != nullptr) {
        const APlanes po = a_planes_view(planes, outer, size, (size + 1023) / 1024);
        CM_LAUNCH("vectorop_kernel", vectorop_planes_kernel<OP>, dim3((unsigned)blocks), dim3(threads), 0, s, a, b,
                  c, size, outer, (uint64_t)a_inc, (uint64_t)b_inc, act, alpha, tab, len, po);
        return CM_OK;
    }
    CM_LAUNCH("vectorop_kernel", vectorop_kernel<OP>, dim3((unsigned)blocks), dim3(threads), 0, s, a, b, c,
                       size, outer, (uint64_t)a_inc, (uint64_t)b_inc, act, alpha, tab, len);
    return CM_OK;
}

}  // namespace

int prepare_softmax(DeviceState* st) {
    const void* fns[] = {
        reinterpret_cast<const void*>(softmax_rows_kernel<1, true>), reinterpret_cast<const void*>(softmax_rows_kernel<2, true>),
        reinterpret_cast<const void*>(softmax_rows_kernel<3, true>), reinterpret_cast<const void*>(softmax_rows_kernel<4, true>),
        reinterpret_cast<const void*>(softmax_rows_kernel<6, true>), reinterpret_cast<const void*>(softmax_rows_kernel<8, true>),
        reinterpret_cast<const void*>(softmax_rows_kernel<1, false>), reinterpret_cast<const void*>(softmax_rows_kernel<2, false>),
        reinterpret_cast<const void*>(softmax_rows_kernel<3, false>), reinterpret_cast<const void*>(softmax_rows_kernel<4, false>),
        reinterpret_cast<const void*>(softmax_rows_kernel<6, false>), reinterpret_cast<const void*>(softmax_rows_kernel<8, false>),
        reinterpret_cast<const void*>(softmax_long_kernel<true>), reinterpret_cast<const void*>(softmax_long_kernel<false>),
        reinterpret_cast<const void*>(softmax_cols_kernel<1, true>), reinterpret_cast<const void*>(softmax_cols_kernel<2, true>),
        reinterpret_cast<const void*>(softmax_cols_kernel<3, true>), reinterpret_cast<const void*>(softmax_cols_kernel<4, true>),
        reinterpret_cast<const void*>(softmax_cols_kernel<6, true>), reinterpret_cast<const void*>(softmax_cols_kernel<8, true>),
        reinterpret_cast<const void*>(softmax_cols_kernel<1, false>), reinterpret_cast<const void*>(softmax_cols_kernel<2, false>),
        reinterpret_cast<const void*>(softmax_cols_kernel<3, false>), reinterpret_cast<const void*>(softmax_cols_kernel<4, false>),
        reinterpret_cast<const void*>(softmax_cols_kernel<6, false>), reinterpret_cast<const void*>(softmax_cols_kernel<8, false>)};
    for (const void* f : fns)
        CM_HIP_CHECK(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)st->lds_per_block));
    for (uint32_t g = 1; g <= kDaMaxG; g++) {
        CM_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(decode_attn_fn<32, true>(g)),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)st->lds_per_block));
        CM_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(decode_attn_fn<64, true>(g)),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)st->lds_per_block));
        CM_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(decode_attn_fn<32>(g)),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)st->lds_per_block));
        CM_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(decode_attn_fn<64>(g)),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)st->lds_per_block));
    }
    return CM_OK;
}

}  // namespace cm

extern "C" int cm_vectorop_planes(const int16_t* a, const int16_t* b, int16_t* c, uint32_t size, uint32_t op,
                                  uint32_t outer, uint32_t a_inc, uint32_t b_inc, uint32_t act, uint32_t alpha,
                                  void* planes, void* stream) {
    using namespace cm;
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    hipStream_t s = as_stream(stream);
    if (op > OP_GELU_TANH) return fail(CM_EINVAL, "vectorop planes: op %u (not a softmax)", op);
    if (act > ACT_GELU_TANH) return fail(CM_EINVAL, "vectorop: act %u", act);
    if (size % 64 || size > 32768 || a_inc + b_inc != size)
        return fail(CM_EINVAL, "vectorop planes: runs of %u (a multiple of 64 up to 32768) onto contiguous rows "
                               "(a_inc + b_inc = %u)", size, a_inc + b_inc);
    if (planes == nullptr) return fail(CM_EINVAL, "vectorop planes: no planes buffer");
    if (outer != 0 && (a == nullptr || (op < OP_RELU && b == nullptr)))
        return fail(CM_EINVAL, "vectorop planes: a null operand");
    if (!aligned16(a) || !aligned16(c) || (op < OP_RELU && !aligned16(b)) || (reinterpret_cast<uintptr_t>(planes) & 255))
        return fail(CM_EALIGN, "vectorop planes: a, b, c 16-byte and planes 256-byte aligned");
    if (outer == 0) return CM_OK;
    uint32_t ja = (op >= OP_LEAKY && op <= OP_GELU_TANH) ? op - (OP_LEAKY - ACT_LEAKY) : act;
    switch (op) {
    case OP_ADD: return launch_ew<OP_ADD>(a, b, c, size, outer, a_inc, b_inc, ja, alpha, st, s, planes);
    case OP_SUB: return launch_ew<OP_SUB>(a, b, c, size, outer, a_inc, b_inc, ja, alpha, st, s, planes);
    case OP_MUL: return launch_ew<OP_MUL>(a, b, c, size, outer, a_inc, b_inc, ja, alpha, st, s, planes);
    case OP_DIV: return launch_ew<OP_DIV>(a, b, c, size, outer, a_inc, b_inc, ja, alpha, st, s, planes);
    case OP_RELU: return launch_ew<OP_RELU>(a, b, c, size, outer, a_inc, b_inc, ja, alpha, st, s, planes);
    case OP_RELU6: return launch_ew<OP_RELU6>(a, b, c, size, outer, a_inc, b_inc, ja, alpha, st, s, planes);
    default: return launch_ew<OP_LEAKY>(a, b, c, size, outer, a_inc, b_inc, ja, alpha, st, s, planes);
    }
}

extern "C" int cm_vectorop(const int16_t* a, const int16_t* b, int16_t* c, uint32_t size,
                           uint32_t op, uint32_t outer, uint32_t a_inc, uint32_t b_inc,
                           uint32_t act, uint32_t alpha, uint32_t smx_cm, uint32_t smx_cfg,
                           uint32_t smx_mask, void* stream) {
    using namespace cm;
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    hipStream_t s = as_stream(stream);
    if (op > OP_SOFTMAX_T) return fail(CM_EINVAL, "vectorop: op %u", op);
    if (size == 0 || outer == 0) return CM_OK;
    if (!aligned16(a) || !aligned16(c) || (op < OP_RELU && !aligned16(b)))
        return fail(CM_EALIGN, "vectorop: a, b and c must be 16-byte aligned");
    if (outer != 0 && size != 0 && (a == nullptr || c == nullptr || (op < OP_RELU && b == nullptr)))
        return fail(CM_EINVAL, "vectorop: a null operand or output");
    if (op == OP_SOFTMAX || op == OP_SOFTMAX_T)
        return launch_softmax(a, c, size, op, outer, a_inc, b_inc, smx_cm, smx_cfg, smx_mask, 1, 0, 0, st, s);
    if ((a_inc & 7) || (b_inc & 7))
        return fail(CM_EALIGN, "vectorop: a_inc %u / b_inc %u not multiples of 8", a_inc, b_inc);
    if (act > ACT_GELU_TANH) return fail(CM_EINVAL, "vectorop: act %u", act);
    uint32_t ja = (op >= OP_LEAKY && op <= OP_GELU_TANH) ? op - (OP_LEAKY - ACT_LEAKY) : act;
    switch (op) {
    case OP_ADD: return launch_ew<OP_ADD>(a, b, c, size, outer, a_inc, b_inc, ja, alpha, st, s);
    case OP_SUB: return launch_ew<OP_SUB>(a, b, c, size, outer, a_inc, b_inc, ja, alpha, st, s);
    case OP_MUL: return launch_ew<OP_MUL>(a, b, c, size, outer, a_inc, b_inc, ja, alpha, st, s);
    case OP_DIV: return launch_ew<OP_DIV>(a, b, c, size, outer, a_inc, b_inc, ja, alpha, st, s);
    case OP_RELU: return launch_ew<OP_RELU>(a, b, c, size, outer, a_inc, b_inc, ja, alpha, st, s);
    case OP_RELU6: return launch_ew<OP_RELU6>(a, b, c, size, outer, a_inc, b_inc, ja, alpha, st, s);
    default: return launch_ew<OP_LEAKY>(a, b, c, size, outer, a_inc, b_inc, ja, alpha, st, s);
    }
}

extern "C" int cm_softmax(const int16_t* a, int16_t* c, uint32_t size, uint32_t op, uint32_t outer,
                          uint32_t a_inc, uint32_t c_inc, uint32_t smx_cm, uint32_t smx_cfg, uint32_t smx_mask,
                          uint32_t batch, uint64_t a_bs, uint64_t c_bs, void* stream) {
    using namespace cm;
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    if (op != OP_SOFTMAX && op != OP_SOFTMAX_T) return fail(CM_EINVAL, "softmax: op %u is not 10 or 11", op);
    if (size == 0 || outer == 0 || batch == 0) return CM_OK;
    return launch_softmax(a, c, size, op, outer, a_inc, c_inc, smx_cm, smx_cfg, smx_mask, batch, a_bs, c_bs, st,
                          as_stream(stream));
}

namespace cm {
namespace {

int decode_attention_run(const int16_t* q, const int16_t* kc, const int16_t* vc, int16_t* o, uint32_t groups,
                         uint32_t g, uint32_t c, uint32_t head_dim, uint32_t smx_cm, uint32_t smx_cfg,
                         uint32_t smx_mask, const DaPrep* pp, hipStream_t s) {
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    if (groups == 0) return CM_OK;
    if (head_dim != 32 && head_dim != 64)
        return fail(CM_EINVAL, "decode attention: head_dim %u (the kernel takes 32 or 64)", head_dim);
    if (g == 0 || g > kDaMaxG) return fail(CM_EINVAL, "decode attention: %u queries per group (1 .. %u)", g, kDaMaxG);
    if (c == 0 || (c & 63) || c > 8192) return fail(CM_EINVAL, "decode attention: %u cache rows (a multiple of 64, <= 8192)", c);
    if (groups > 0x7FFFFFFFu) return fail(CM_EINVAL, "decode attention: %u groups", groups);
    if (!aligned16(q) || !aligned16(kc) || !aligned16(vc) || !aligned16(o))
        return fail(CM_EALIGN, "decode attention: q, the caches and o must be 16-byte aligned");
    SmxRegs r{smx_cm & 0xFFFFFFu, smx_cfg & 63u, (smx_cfg >> 8) & 31u, smx_mask & 0xFFFFu, smx_mask >> 16, 0};
    r.dlim = smx_dlim(r.cm, r.cs);
    const size_t lds = 4 * (4096 + kDaMaxG * 32 + 2 * kDaWaves * kDaMaxG + kDaMaxG * 64) + (size_t)2 * g * c;
    if (lds > st->lds_per_block) return fail(CM_EINVAL, "decode attention: %zu bytes of LDS", lds);
    const DecodeAttnFn fn = pp != nullptr ? (head_dim == 64 ? decode_attn_fn<64, true>(g) : decode_attn_fn<32, true>(g))
                                          : (head_dim == 64 ? decode_attn_fn<64>(g) : decode_attn_fn<32>(g));
    CM_LAUNCH("decode_attn_kernel", fn, dim3(groups), dim3(kDaThreads), lds, s, q, kc, vc, o, c, r,
              reinterpret_cast<const int4*>(st->smx_tab), pp != nullptr ? *pp : DaPrep{});
    return CM_OK;
}

}  // namespace
}  // namespace cm

extern "C" int cm_decode_attention(const int16_t* q, const int16_t* kc, const int16_t* vc, int16_t* o,
                                   uint32_t groups, uint32_t g, uint32_t c, uint32_t head_dim, uint32_t smx_cm,
                                   uint32_t smx_cfg, uint32_t smx_mask, void* stream) {
    return cm::decode_attention_run(q, kc, vc, o, groups, g, c, head_dim, smx_cm, smx_cfg, smx_mask, nullptr,
                                    cm::as_stream(stream));
}

extern "C" int cm_decode_attention_prep(const int16_t* q, const int16_t* k, const int16_t* v, int16_t* qr,
                                        int16_t* kc, int16_t* vc, int16_t* o, uint32_t batch, uint32_t heads,
                                        uint32_t kv_heads, uint32_t head_dim, uint32_t cache_rows, uint32_t pos,
                                        const void* rope_row, const void* params_q, uint32_t op_q,
                                        const void* params_k, uint32_t op_k, uint32_t smx_cm, uint32_t smx_cfg,
                                        uint32_t smx_mask, void* stream) {
    using namespace cm;
    if (batch == 0) return CM_OK;
    if (kv_heads == 0 || heads % kv_heads) return fail(CM_EINVAL, "decode attention: %u heads over %u KV heads", heads, kv_heads);
    if (pos >= cache_rows) return fail(CM_EINVAL, "decode attention: position %u of %u cache rows", pos, cache_rows);
    for (uint32_t op : {op_q, op_k})
        if ((op & 15) != ro::RO_ROPE || ((op >> 4) & 3) != 0 || ((op >> 8) & 3) != 0 || (op & ro::F_P_KEEP))
            return fail(CM_EINVAL, "decode attention: 0x%x is not an int16 ROPE job's op word", op);
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(qr) || !aligned16(rope_row) ||
        (reinterpret_cast<uintptr_t>(params_q) & 15) || (reinterpret_cast<uintptr_t>(params_k) & 15))
        return fail(CM_EALIGN, "decode attention: the prep's operands are not aligned");
    const DaPrep pp{q, k, v, qr, kc, vc, static_cast<const int32_t*>(rope_row), static_cast<const uint8_t*>(params_q),
                    static_cast<const uint8_t*>(params_k), (op_q & ro::F_P_BCAST) ? 1u : 0u,
                    (op_k & ro::F_P_BCAST) ? 1u : 0u, kv_heads, pos};
    return decode_attention_run(qr, kc, vc, o, batch * kv_heads, heads / kv_heads, cache_rows, head_dim, smx_cm,
                                smx_cfg, smx_mask, &pp, as_stream(stream));
}
