// cm_rowops.hip -- the RowOps unit: one job of the register contract of
// doc/kernels/ROWOPS_RTL_KERNEL.md section 1 with the integer specifications of
// inference-scheduler/src/rowops_spec.py.
//
// Kernels:
//   * stream ops (COPY, ADDX, DEQUANT, MULACT, GATE) and ROPE: one thread per 16-byte
//     output word, so a wavefront writes 1 KiB of a row per instruction;
//   * NORM: one wavefront per row -- exact S1 (int64) and S2 (128-bit) by wavefront
//     reductions, then the table + Newton reciprocal square root and a second pass;
//   * TRANSPOSE, FOLD: one thread per output element.
// The sigmoid and rsqrt tables are read from the device's 64 KiB table image (built at
// init, replaced by a TLOAD job), the parameter block from the device's parameter RAM.
#include "cm_common.h"
#include "cm_rowops_math.h"

#include <algorithm>

namespace cm {
namespace {

using namespace ro;

struct Job {
    const uint8_t* a;
    const uint8_t* b;
    uint8_t* c;
    uint32_t op, n, c1, c2, a_s1, a_s2, b_s1, b_s2, c_s1, c_s2;
    i64 eps;
    uint32_t aux, bq_sh, win_lo, win_hi;
};

// float32(v * 2^-sh) rounded to nearest even: v is exact in double (|v| < 2^32), one
// rounding to float.
__device__ __forceinline__ uint32_t dequant_bits(i64 v, int sh) {
    const float f = (float)ldexp((double)v, -sh);
    return __float_as_uint(f);
}

// ---------------------------------------------------------------- parameter load
// A job that loads parameters copies its block (n entries, or entry 0 with P_BCAST) into the
// parameter RAM; workgroup 0 of the job kernel does it while the job reads `p` itself.
__device__ __forceinline__ void pram_load(const uint8_t* p, uint8_t* pram, uint32_t entries) {
    if (pram == nullptr || blockIdx.x != 0 || blockIdx.y != 0) return;
    for (uint32_t i = threadIdx.x; i < entries; i += blockDim.x)
        *reinterpret_cast<uint4*>(pram + 16u * i) = *reinterpret_cast<const uint4*>(p + 16u * i);
}

// ---------------------------------------------------------------- stream ops + ROPE
__global__ __launch_bounds__(256) void ro_stream_kernel(Job j, const uint8_t* __restrict__ params,
                                                        uint8_t* pram_dst, uint32_t p_entries,
                                                        bool bcast, const uint8_t* __restrict__ tab) {
    pram_load(params, pram_dst, p_entries);
    const uint32_t code = j.op & 15, ak = (j.op >> 4) & 3, bk = (j.op >> 6) & 3;
    const uint32_t ck = code == RO_DEQUANT ? 2u : ((j.op >> 8) & 3);
    const uint32_t abytes = ak == 0 ? 2 : 4, bbytes = bk == 0 ? 2 : 4, cbytes = ck == 0 ? 2 : 4;
    const uint32_t lanes = 16 / cbytes;
    const uint32_t words = (j.n * cbytes + 15) / 16;
    const u64 total = (u64)words * j.c1 * j.c2;
    const bool ben = (j.op & F_B_EN) != 0;
    for (u64 w = (u64)blockIdx.x * blockDim.x + threadIdx.x; w < total; w += (u64)gridDim.x * blockDim.x) {
        const uint32_t wi = (uint32_t)(w % words);
        const u64 row = w / words;
        const uint32_t i1 = (uint32_t)(row % j.c1), i2 = (uint32_t)(row / j.c1);
        const uint8_t* ra = j.a + (u64)i2 * j.a_s2 + (u64)i1 * j.a_s1;
        const uint8_t* rb = j.b + (u64)i2 * j.b_s2 + (u64)i1 * j.b_s1;
        uint8_t* rc = j.c + (u64)i2 * j.c_s2 + (u64)i1 * j.c_s1;
        const bool zero_a = (code == RO_COPY || code == RO_ADDX) && (i1 < j.win_lo || i1 >= j.win_hi);
        uint32_t out[4] = {0, 0, 0, 0};
        for (uint32_t l = 0; l < lanes; l++) {
            const uint32_t col = wi * lanes + l;
            if (col >= j.n) break;
            const Param q = ld_param(params, col, bcast);
            i64 r = 0;
            if (code == RO_ROPE) {
                r = rope_value(reinterpret_cast<const int16_t*>(ra), col, j.aux & 0xFFF,
                               reinterpret_cast<const int32_t*>(rb), q);
            } else {
                const i64 x = zero_a ? 0 : ld_kind(ra + (u64)abytes * col, ak);
                const i64 y = (ben && code != RO_DEQUANT) ? ld_kind(rb + (u64)bbytes * col, bk) : 0;
                if (code == RO_COPY || code == RO_ADDX) {
                    r = copy_addx(x, y, q, j.op, j.bq_sh, ck);
                } else if (code == RO_DEQUANT) {
                    r = (i64)dequant_bits(x, q.sc);
                } else if (code == RO_GATE) {
                    const i64 th = 2 * sig_q(x << q.sa, tab) - ((i64)1 << 24);
                    const i64 sg = sig_q(y << q.sb, tab);
                    r = sat16(rne_shr((i128)th * sg, q.sc));
                } else {   // MULACT
                    r = sat16(rne_shr((i128)silu_q(x << q.sa, tab) * y, q.sc));
                }
            }
            if (cbytes == 2) out[l >> 1] |= ((uint32_t)(uint16_t)r) << (16 * (l & 1));
            else out[l] = (uint32_t)r;
        }
        *reinterpret_cast<uint4*>(rc + 16u * wi) = make_uint4(out[0], out[1], out[2], out[3]);
    }
}

// ---------------------------------------------------------------- NORM
__device__ __forceinline__ i128 wave_sum128(i128 v) {
    u64 lo = (u64)v, hi = (u64)(v >> 64);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        u64 olo = __shfl_xor(lo, off, 64), ohi = __shfl_xor(hi, off, 64);
        u64 nlo = lo + olo;
        hi = hi + ohi + (nlo < lo ? 1 : 0);
        lo = nlo;
    }
    return (i128)(((unsigned __int128)hi << 64) | lo);
}

__global__ __launch_bounds__(256) void ro_norm_kernel(Job j, const uint8_t* __restrict__ params,
                                                      uint8_t* pram_dst, uint32_t p_entries, bool bcast,
                                                      const uint8_t* __restrict__ tab) {
    pram_load(params, pram_dst, p_entries);
    const uint32_t lane = threadIdx.x & 63;
    const u64 row = (u64)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= (u64)j.c1 * j.c2) return;
    const uint32_t i1 = (uint32_t)(row % j.c1), i2 = (uint32_t)(row / j.c1);
    const uint32_t ak = (j.op >> 4) & 3, abytes = ak == 0 ? 2 : 4;
    const uint8_t* ra = j.a + (u64)i2 * j.a_s2 + (u64)i1 * j.a_s1;
    uint8_t* rc = j.c + (u64)i2 * j.c_s2 + (u64)i1 * j.c_s1;
    const bool ln = (j.op & F_NORM_LN) != 0;
    i64 s1 = 0;
    i128 s2 = 0;
    for (uint32_t col = lane; col < j.n; col += 64) {
        const i64 x = ld_kind(ra + (u64)abytes * col, ak);
        s1 += x;
        s2 += (i128)(x * x);      // |x| < 2^31: x^2 < 2^62 fits an int64
    }
    for (int off = 32; off > 0; off >>= 1) s1 += __shfl_xor(s1, off, 64);
    const i128 S1 = s1, S2 = wave_sum128(s2);
    i128 D = ln ? ((i128)j.n * S2 - S1 * S1 + (i128)j.eps) : (S2 + (i128)j.eps);
    if (D <= 0) D = 1;
    u64 Rm;
    int sh;
    rsqrt_bf(D, Rm, sh, tab);
    const uint32_t words = (j.n * 2 + 15) / 16;
    for (uint32_t wi = lane; wi < words; wi += 64) {
        uint32_t out[4] = {0, 0, 0, 0};
        for (uint32_t l = 0; l < 8; l++) {
            const uint32_t col = wi * 8 + l;
            if (col >= j.n) break;
            const Param q = ld_param(params, col, bcast);
            const i64 x = ld_kind(ra + (u64)abytes * col, ak);
            const i128 A = ln ? ((i128)j.n * x - S1) : (i128)x;
            const i128 P1 = (A * (i128)Rm) >> (sh - 24);
            const i128 s = P1 * (i128)q.g + ((i128)q.bq << j.bq_sh);
            out[l >> 1] |= ((uint32_t)(uint16_t)sat16(rne_shr(s, q.sc))) << (16 * (l & 1));
        }
        *reinterpret_cast<uint4*>(rc + 16u * wi) = make_uint4(out[0], out[1], out[2], out[3]);
    }
}

// ---------------------------------------------------------------- fast NORM / COPY / ADDX
// Rows of whole 8-element units with 16-byte aligned rows: the parameter block staged once per
// workgroup in LDS, 16-byte loads and stores, and 64-bit arithmetic wherever it is exact
// (checked per row or per element), the 128-bit forms above otherwise.

// The 8 elements of unit u of a row (int16 or int32 lanes) as int32.
template <int K>
__device__ __forceinline__ void ld_unit(const uint8_t* row, uint32_t u, int (&x)[8]) {
    if constexpr (K == 0) {
        const int4 w = *reinterpret_cast<const int4*>(row + 16u * u);
        const int16_t* h = reinterpret_cast<const int16_t*>(&w);
#pragma unroll
        for (int l = 0; l < 8; l++) x[l] = h[l];
    } else {
        const int4 w0 = *reinterpret_cast<const int4*>(row + 32u * u);
        const int4 w1 = *reinterpret_cast<const int4*>(row + 32u * u + 16);
        x[0] = w0.x; x[1] = w0.y; x[2] = w0.z; x[3] = w0.w;
        x[4] = w1.x; x[5] = w1.y; x[6] = w1.z; x[7] = w1.w;
    }
}

__device__ __forceinline__ void stage_params(uint4* lds, const uint8_t* params, uint32_t entries, uint32_t units) {
    for (uint32_t i = threadIdx.x; i < entries; i += blockDim.x)
        lds[pslot(i, units)] = reinterpret_cast<const uint4*>(params)[i];
    __syncthreads();
}

// COPY / ADDX parameters as the element loop uses them, one 16-byte entry per column: the
// three shifts and two fast-path flags in one word (sa | sb << 8 | sc << 16; bit 24: every
// term within the 64-bit bounds with a 32-bit B, bit 25: with a 16-bit B), G, and
// Bq 2^bq_sh + 2^(sc - 1) (the bias with the rounding half folded in; 0 when bq_sh > 40, a
// job the 128-bit path takes whole).
template <uint32_t BATCH = 1>
__device__ __forceinline__ void stage_addx_params(uint4* lds, const uint8_t* params, uint32_t entries, uint32_t units,
                                                  uint32_t bq_sh) {
    stage_entries<BATCH>(params, entries, [&](uint32_t i, const uint4& raw) {
        const Param q = param_of(raw);
        const bool base = q.sa <= 30 && q.sc <= 61;
        const uint32_t w = (uint32_t)q.sa | ((uint32_t)q.sb << 8) | ((uint32_t)q.sc << 16) |
                           ((base && q.sb <= 30) ? 1u << 24 : 0u) | ((base && q.sb <= 46) ? 1u << 25 : 0u);
        const u64 bs = bq_sh <= 40 ? (u64)(q.bq * ((i64)1 << bq_sh) + norm_half((uint32_t)q.sc)) : 0;
        lds[pslot(i, units)] = make_uint4(w, (uint32_t)q.g, (uint32_t)bs, (uint32_t)(bs >> 32));
    });
}

// One COPY / ADDX unit in 128-bit arithmetic (the scale flag, or shifts past the 64-bit
// bounds), from the job's own parameter block in global memory.
__device__ __forceinline__ void addx_unit_wide(const int (&x)[8], const int (&y)[8], bool ben, int ck, uint32_t u,
                                            uint32_t bq_sh, bool scale, const uint8_t* praw, bool bcast, int (&r)[8]) {
    for (int l = 0; l < 8; l++) {
        const Param q = ld_param(praw, 8 * u + l, bcast);
        const i128 s = ((i128)x[l] << q.sa) + ((i128)(ben ? y[l] : 0) << q.sb) + ((i128)q.bq << bq_sh);
        const i128 v = rne_shr(scale ? s * (i128)q.g : s, q.sc);
        r[l] = (int)(ck == 0 ? sat16(v) : sat32(v));
    }
}

// One COPY / ADDX unit from the staged entries (stage_addx_params): 64-bit arithmetic where
// every term stays below 2^61 (x << sa <= 2^61, y << sb, Bq << bq_sh <= 2^61), round half to even
// as one shift and an exact-tie test; else the 128-bit form (a branch taken by the lanes that
// need it).
template <int BK, int CK, bool BEN>
__device__ __forceinline__ void addx_unit(const int (&x)[8], const int (&y)[8], uint32_t u, uint32_t units,
                                          const Job& j, const uint4* ro_lds, const uint8_t* praw, bool bcast,
                                          bool scale, bool relu, int (&r)[8]) {
    bool wide = scale || j.bq_sh > 40;
#pragma unroll
    for (int l = 0; l < 8; l++) {
        const uint4 e = ro_lds[bcast ? 0u : l * units + u];
        const uint32_t sa = e.x & 63, sb = (e.x >> 8) & 63, sc = (e.x >> 16) & 63;
        wide |= ((e.x >> (BK == 0 ? 25 : 24)) & 1) == 0;
        const i64 yv = BEN ? (i64)y[l] : 0;
        // shifts on the unsigned images (defined for negative operands; exact within the bounds)
        const i64 w = (i64)(((u64)(i64)x[l] << (sa & 31)) + ((u64)yv << sb) + (((u64)e.w << 32) | e.z));
        i64 v = w >> sc;
        v &= ~(i64)((u64)w << ((64 - sc) & 63) == 0);
        v = CK == 0 ? (v > 32767 ? 32767 : (v < -32768 ? -32768 : v))
                    : (v > 2147483647 ? 2147483647 : (v < -2147483647LL - 1 ? -2147483647LL - 1 : v));
        r[l] = (int)v;
    }
    if (__any(wide)) {
        if (wide) addx_unit_wide(x, y, BEN, CK, u, j.bq_sh, scale, praw, bcast, r);
    }
    if (relu) {
#pragma unroll
        for (int l = 0; l < 8; l++) r[l] = r[l] < 0 ? 0 : r[l];
    }
}

// One NORM row of the fast path (norm_row_vals), its int16 results to rc (null: not written) and, with PL, their
// byte planes and row sums per 1024 columns (unit u in sum u / 128 = k / 2) as row `prow` of
// `po`.  Wavefront-uniform control.
template <int UPL, bool PL>
__device__ __forceinline__ void norm_row(const Job& j, const int (&x)[UPL][8], uint8_t* rc, const uint4* ro_lds,
                                         bool bcast, const uint8_t* tab, uint32_t lane, uint32_t units, bool ln,
                                         const APlanes& po, u64 prow) {
    int4 o[UPL];
    norm_row_vals<UPL>(j.n, j.eps, x, ro_lds, bcast, tab, lane, units, ln, o);
    int32_t ps[UPL];
#pragma unroll
    for (int k = 0; k < UPL; k++) {
        const uint32_t u = lane + 64 * k;
        ps[k] = 0;
        if (u >= units) continue;
        if (rc != nullptr) store_stream(rc + 16u * u, o[k]);
        if constexpr (PL) {
            uint2 h, l;
            split8(o[k], h, l);
            *reinterpret_cast<uint2*>(po.hi + prow * po.k + 8u * u) = h;
            *reinterpret_cast<uint2*>(po.lo + prow * po.k + 8u * u) = l;
            ps[k] = sum8(o[k]);
        }
    }
    if constexpr (PL) {
#pragma unroll
        for (int sl = 0; sl < (UPL + 1) / 2; sl++) {
            int32_t v = ps[2 * sl] + (2 * sl + 1 < UPL ? ps[2 * sl + 1] : 0);
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
            if (lane == 0 && (uint32_t)sl < po.nsum) po.part[(u64)sl * po.lines + prow] = v;
        }
    }
}

// NORM: a wavefront per row (rows in turn over the grid), the row held in registers between
// the sums and the output: UPL units of 8 elements per lane, n <= 512 UPL.  With ADDX the row
// is first the output of the COPY / ADDX job `ja` (int32, AK int32 or int16 A, int16 B, its
// parameters staged after the NORM's), stored to ja.c and normalised from the registers: the
// two-job chain ADDX -> NORM with one read of each row.  PL: the byte planes of the output.
template <int AK, int UPL, bool ADDX, bool PL, int NW>
__global__ __launch_bounds__(64 * NW) void ro_norm_fast_kernel(Job j, const uint8_t* __restrict__ params,
                                                           uint8_t* pram_dst, uint32_t p_entries, bool bcast,
                                                           const uint8_t* __restrict__ tab, Job ja,
                                                           const uint8_t* __restrict__ pa, bool bca, APlanes po) {
    extern __shared__ __attribute__((aligned(16))) uint4 ro_lds[];
    const uint32_t lane = threadIdx.x & 63;
    const u64 rows = (u64)j.c1 * j.c2;
    const bool ln = (j.op & F_NORM_LN) != 0;
    const uint32_t units = j.n / 8;
    const u64 stride = (u64)gridDim.x * (blockDim.x >> 6);
    const uint32_t nsl = bcast ? 1u : j.n;
    uint4* a_lds = ro_lds + nsl;                          // the ADDX job's parameters
    int x[UPL][8];
    int4 yw[UPL];                                         // the ADDX job's int16 B, unpacked at use
    auto load_row = [&](u64 row) {
        const Job& jl = ADDX ? ja : j;
        const uint32_t i1 = (uint32_t)(row % jl.c1), i2 = (uint32_t)(row / jl.c1);
        const uint8_t* ra = jl.a + (u64)i2 * jl.a_s2 + (u64)i1 * jl.a_s1;
#pragma unroll
        for (int k = 0; k < UPL; k++) {
            const uint32_t u = lane + 64 * k;
            if (u < units) {
                ld_unit<AK>(ra, u, x[k]);
                if constexpr (ADDX)
                    yw[k] = *reinterpret_cast<const int4*>(ja.b + (u64)i2 * ja.b_s2 + (u64)i1 * ja.b_s1 + 16u * u);
            } else {
#pragma unroll
                for (int l = 0; l < 8; l++) x[k][l] = 0;
                yw[k] = make_int4(0, 0, 0, 0);
            }
        }
    };
    u64 row = (u64)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row < rows) load_row(row);                       // in flight while the parameters are staged
    pram_load(params, pram_dst, p_entries);
    if constexpr (ADDX) {
        stage_addx_params(a_lds, pa, bca ? 1u : ja.n, units, ja.bq_sh);
    }
    stage_norm_params(ro_lds, params, nsl, units, j.bq_sh);
    __syncthreads();
    const bool scale = (ja.op & F_SCALE) != 0, relu = (ja.op & F_RELU) != 0;
    for (; row < rows; row += stride) {
        const uint32_t i1 = (uint32_t)(row % j.c1), i2 = (uint32_t)(row / j.c1);
        if constexpr (ADDX) {
            // the ADDX outputs (int32) replace the row in registers and go to ja.c
            uint8_t* rc1 = ja.c + (u64)i2 * ja.c_s2 + (u64)i1 * ja.c_s1;
#pragma unroll
            for (int k = 0; k < UPL; k++) {
                const uint32_t u = lane + 64 * k;
                if (u >= units) continue;
                int r[8], y[8];
                const int16_t* yh = reinterpret_cast<const int16_t*>(&yw[k]);
#pragma unroll
                for (int l = 0; l < 8; l++) y[l] = yh[l];
                addx_unit<0, 1, true>(x[k], y, u, units, ja, a_lds, pa, bca, scale, relu, r);
                store_stream(rc1 + 32u * u, make_int4(r[0], r[1], r[2], r[3]));
                store_stream(rc1 + 32u * u + 16, make_int4(r[4], r[5], r[6], r[7]));
#pragma unroll
                for (int l = 0; l < 8; l++) x[k][l] = r[l];
            }
        }
        norm_row<UPL, PL>(j, x, j.c != nullptr ? j.c + (u64)i2 * j.c_s2 + (u64)i1 * j.c_s1 : nullptr, ro_lds, bcast, tab,
                          lane, units, ln, po,
                          row);
        if (row + stride < rows) load_row(row + stride);
    }
}

// NORM with a workgroup of TPR threads per row (rows in turn over the grid): UPL units of 8
// elements per thread (n <= 8 TPR UPL), the wavefronts' sums added through LDS.  A wavefront per
// row leaves each lane a long serial chain of 64-bit arithmetic over several units at a few
// wavefronts per SIMD; here a lane holds one or two units and a row has TPR / 64 wavefronts.
// ADDX and PL as in ro_norm_fast_kernel: the residual add's int32 output formed in registers,
// stored and normalised; the output's byte planes and per-slab row sums for the next GEMM.
template <int AK, int UPL, bool ADDX, bool PL, int TPR>
__global__ __launch_bounds__(TPR) void ro_norm_wg_kernel(Job j, const uint8_t* __restrict__ params, uint8_t* pram_dst,
                                                         uint32_t p_entries, bool bcast,
                                                         const uint8_t* __restrict__ tab, Job ja,
                                                         const uint8_t* __restrict__ pa, bool bca, APlanes po) {
    constexpr int NWV = TPR / 64;
    extern __shared__ __attribute__((aligned(16))) uint4 ro_lds[];
    __shared__ NormSums wsum[2][NWV];
    __shared__ int32_t slab_acc[2][4];                   // a row's slab sums (n <= 4096)
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const u64 rows = (u64)j.c1 * j.c2;
    const bool ln = (j.op & F_NORM_LN) != 0;
    const uint32_t units = j.n / 8;
    const uint32_t nsl = bcast ? 1u : j.n;
    uint4* a_lds = ro_lds + nsl;                         // the ADDX job's parameters
    int x[UPL][8], y[UPL][8];
    auto load_row = [&](u64 row) {
        const Job& jl = ADDX ? ja : j;
        const uint32_t i1 = (uint32_t)(row % jl.c1), i2 = (uint32_t)(row / jl.c1);
        const uint8_t* ra = jl.a + (u64)i2 * jl.a_s2 + (u64)i1 * jl.a_s1;
#pragma unroll
        for (int k = 0; k < UPL; k++) {
            const uint32_t u = t + TPR * k;
            if (u < units) {
                ld_unit<AK>(ra, u, x[k]);
                if constexpr (ADDX) ld_unit<0>(ja.b + (u64)i2 * ja.b_s2 + (u64)i1 * ja.b_s1, u, y[k]);
            } else {
#pragma unroll
                for (int l = 0; l < 8; l++) x[k][l] = y[k][l] = 0;
            }
        }
    };
    u64 row = blockIdx.x;
    if (row < rows) load_row(row);                       // in flight while the parameters are staged
    pram_load(params, pram_dst, p_entries);
    // A plain NORM: each lane stages the entries of its own units (the only slots it reads,
    // norm_row_finish / norm_unit_wide), so no barrier waits for the staging; their loads go
    // out here beside the row's and are decoded after the row's sums.
    constexpr bool SELF = !ADDX && !PL;
    uint4 praw[SELF ? UPL : 1][SELF ? 8 : 1];
    if constexpr (SELF) {
        const uint4* src = reinterpret_cast<const uint4*>(params);
#pragma unroll
        for (int k = 0; k < UPL; k++) {
            const uint32_t u = t + TPR * k;
#pragma unroll
            for (int l = 0; l < 8; l++)
                praw[k][l] = u < units ? src[bcast ? 0u : 8u * u + l] : make_uint4(0, 0, 0, 0);
        }
    } else {
        // few rows a workgroup: the staging's memory latency is on the critical path, so each
        // thread's entries are loaded four at a time
        if constexpr (ADDX) {
            stage_addx_params<4>(a_lds, pa, bca ? 1u : ja.n, units, ja.bq_sh);
        }
        stage_norm_params<4>(ro_lds, params, nsl, units, j.bq_sh);
        if (t < 8) slab_acc[t >> 2][t & 3] = 0;
        __syncthreads();
    }
    const bool scale = (ja.op & F_SCALE) != 0, relu = (ja.op & F_RELU) != 0;
    const uint32_t nslab = min(po.nsum, (units + 127) / 128);
    for (uint32_t it = 0; row < rows; row += gridDim.x, it++) {
        const uint32_t i1 = (uint32_t)(row % j.c1), i2 = (uint32_t)(row / j.c1);
        if constexpr (ADDX) {
            // the ADDX outputs (int32) replace the row in registers and go to ja.c
            uint8_t* rc1 = ja.c + (u64)i2 * ja.c_s2 + (u64)i1 * ja.c_s1;
#pragma unroll
            for (int k = 0; k < UPL; k++) {
                const uint32_t u = t + TPR * k;
                if (u >= units) continue;
                int r[8];
                addx_unit<0, 1, true>(x[k], y[k], u, units, ja, a_lds, pa, bca, scale, relu, r);
                store_stream(rc1 + 32u * u, make_int4(r[0], r[1], r[2], r[3]));
                store_stream(rc1 + 32u * u + 16, make_int4(r[4], r[5], r[6], r[7]));
#pragma unroll
                for (int l = 0; l < 8; l++) x[k][l] = r[l];
            }
        }
        NormSums ts = norm_sums<UPL>(x);
        norm_sums_wave(ts);
        if constexpr (SELF) {
            if (it == 0) {
#pragma unroll
                for (int k = 0; k < UPL; k++) {
                    const uint32_t u = t + TPR * k;
                    if (u >= units) continue;
#pragma unroll
                    for (int l = 0; l < 8; l++) {
                        const uint32_t i = bcast ? 0u : 8u * u + l;
                        if (bcast && l > 0) break;
                        norm_entry(ro_lds, i, praw[k][l], units, j.bq_sh);
                    }
                }
            }
        }
        NormSums* ws = wsum[it & 1];                     // alternate: a row's reads end before the next's writes
        if (lane == 0) ws[wave] = ts;
        __syncthreads();
        ts = ws[0];
#pragma unroll
        for (int w = 1; w < NWV; w++) norm_sums_add(ts, ws[w]);
        int4 o[UPL];
        norm_row_finish<UPL>(j.n, j.eps, ts, x, ro_lds, bcast, tab, t, TPR, units, ln, o);
        uint8_t* rc = j.c != nullptr ? j.c + (u64)i2 * j.c_s2 + (u64)i1 * j.c_s1 : nullptr;   // null: planes alone
#pragma unroll
        for (int k = 0; k < UPL; k++) {
            const uint32_t u = t + TPR * k;
            if (u < units && rc != nullptr) store_stream(rc + 16u * u, o[k]);
        }
        if constexpr (PL) {
            int32_t* sa = slab_acc[it & 1];
#pragma unroll
            for (int k = 0; k < UPL; k++) {
                const uint32_t u = t + TPR * k;
                int32_t v = 0;
                if (u < units) {
                    uint2 h, l;
                    split8(o[k], h, l);
                    *reinterpret_cast<uint2*>(po.hi + row * po.k + 8u * u) = h;
                    *reinterpret_cast<uint2*>(po.lo + row * po.k + 8u * u) = l;
                    v = sum8(o[k]);
                }
#pragma unroll
                for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
                // a wavefront's 64 units lie in one 128-unit slab (1024 elements)
                const uint32_t u0 = wave * 64 + TPR * k;
                if (lane == 0 && u0 < units) atomicAdd(&sa[u0 / 128], v);
            }
            __syncthreads();
            if (t < nslab) {
                po.part[(u64)t * po.lines + row] = sa[t];
                sa[t] = 0;                               // for the row after next
            }
        }
        if (row + gridDim.x < rows) load_row(row + gridDim.x);
    }
}

// COPY / ADDX: a lane per 8-element unit of a row (units in turn over the grid).
template <int AK, int BK, int CK, bool BEN>
__global__ __launch_bounds__(256) void ro_addx_fast_kernel(Job j, const uint8_t* __restrict__ params,
                                                           uint8_t* pram_dst, uint32_t p_entries, bool bcast) {
    extern __shared__ __attribute__((aligned(16))) uint4 ro_lds[];
    pram_load(params, pram_dst, p_entries);
    const uint32_t units = j.n / 8;
    stage_addx_params(ro_lds, params, bcast ? 1u : j.n, units, j.bq_sh);
    __syncthreads();
    const u64 total = (u64)units * j.c1 * j.c2;
    const bool scale = (j.op & F_SCALE) != 0, relu = (j.op & F_RELU) != 0;
    for (u64 w = (u64)blockIdx.x * blockDim.x + threadIdx.x; w < total; w += (u64)gridDim.x * blockDim.x) {
        const uint32_t u = (uint32_t)(w % units);
        const u64 row = w / units;
        const uint32_t i1 = (uint32_t)(row % j.c1), i2 = (uint32_t)(row / j.c1);
        const bool zero_a = i1 < j.win_lo || i1 >= j.win_hi;
        int x[8], y[8];
        if (zero_a) {
#pragma unroll
            for (int l = 0; l < 8; l++) x[l] = 0;
        } else {
            ld_unit<AK>(j.a + (u64)i2 * j.a_s2 + (u64)i1 * j.a_s1, u, x);
        }
        if constexpr (BEN) ld_unit<BK>(j.b + (u64)i2 * j.b_s2 + (u64)i1 * j.b_s1, u, y);
        int r[8];
        addx_unit<BK, CK, BEN>(x, y, u, units, j, ro_lds, params, bcast, scale, relu, r);
        uint8_t* rc = j.c + (u64)i2 * j.c_s2 + (u64)i1 * j.c_s1;
        if constexpr (CK == 0) {
            int4 o;
            o.x = (int)((uint32_t)(uint16_t)r[0] | ((uint32_t)(uint16_t)r[1] << 16));
            o.y = (int)((uint32_t)(uint16_t)r[2] | ((uint32_t)(uint16_t)r[3] << 16));
            o.z = (int)((uint32_t)(uint16_t)r[4] | ((uint32_t)(uint16_t)r[5] << 16));
            o.w = (int)((uint32_t)(uint16_t)r[6] | ((uint32_t)(uint16_t)r[7] << 16));
            store_stream(rc + 16u * u, o);
        } else {
            store_stream(rc + 32u * u, make_int4(r[0], r[1], r[2], r[3]));
            store_stream(rc + 32u * u + 16, make_int4(r[4], r[5], r[6], r[7]));
        }
    }
}

// ---------------------------------------------------------------- fast DEQUANT / MULACT / GATE / ROPE
// The stream ops over rows of whole 8-element units with 16-byte aligned rows: a lane per unit
// (units in turn over the grid), the parameter block staged in LDS, 16-byte loads and stores,
// 64-bit arithmetic where an element's shifts keep every term below 2^62 (sa, sb <= 23 with
// int16 operands, sc <= 61), the 128-bit rule of ro_stream_kernel otherwise.  DEQUANT goes
// through float: float(x) 2^-sc is the double route's one rounding (the scaling is exact for
// |x| < 2^31 and sc <= 63).  ROPE: the unit's rotate-half partner is the unit HD / 2 columns
// away in the same head (HD a multiple of 16), the table row's cos / sin 8 at a time.  MULACT and
// GATE come here with B enabled (int16).

template <uint32_t CODE>
__global__ __launch_bounds__(256) void ro_unit_fast_kernel(Job j, const uint8_t* __restrict__ params,
                                                           uint8_t* pram_dst, uint32_t p_entries, bool bcast,
                                                           const uint8_t* __restrict__ tab) {
    extern __shared__ __attribute__((aligned(16))) uint4 ro_lds[];
    pram_load(params, pram_dst, p_entries);
    const uint32_t units = j.n / 8;
    stage_params(ro_lds, params, bcast ? 1u : j.n, units);
    const u64 total = (u64)units * j.c1 * j.c2;
    const uint32_t HD = j.aux & 0xFFF, half = HD / 2;
    for (u64 w = (u64)blockIdx.x * blockDim.x + threadIdx.x; w < total; w += (u64)gridDim.x * blockDim.x) {
        const uint32_t u = (uint32_t)(w % units);
        const u64 row = w / units;
        const uint32_t i1 = (uint32_t)(row % j.c1), i2 = (uint32_t)(row / j.c1);
        const uint8_t* ra = j.a + (u64)i2 * j.a_s2 + (u64)i1 * j.a_s1;
        const uint8_t* rb = j.b + (u64)i2 * j.b_s2 + (u64)i1 * j.b_s1;
        uint8_t* rc = j.c + (u64)i2 * j.c_s2 + (u64)i1 * j.c_s1;
        int x[8];
        ld_unit<0>(ra, u, x);
        if constexpr (CODE == RO_DEQUANT) {
            float f[8];
#pragma unroll
            for (int l = 0; l < 8; l++) {
                const Param q = param_of(ro_lds[bcast ? 0u : l * units + u]);
                f[l] = ldexpf((float)x[l], -q.sc);
            }
            store_stream(rc + 32u * u, *reinterpret_cast<const int4*>(f));
            store_stream(rc + 32u * u + 16, *reinterpret_cast<const int4*>(f + 4));
            continue;
        }
        int r[8];
        if constexpr (CODE == RO_ROPE) {
            const uint32_t d0 = (8 * u) % HD;
            const bool lo = d0 < half;
            int p[8];
            ld_unit<0>(ra, lo ? u + half / 8 : u - half / 8, p);
            const int4 c0 = *reinterpret_cast<const int4*>(rb + 4u * d0);
            const int4 c1 = *reinterpret_cast<const int4*>(rb + 4u * d0 + 16);
            const int4 s0 = *reinterpret_cast<const int4*>(rb + 4u * (HD + d0));
            const int4 s1 = *reinterpret_cast<const int4*>(rb + 4u * (HD + d0) + 16);
            const int cs[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
            const int sn[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
            for (int l = 0; l < 8; l++) {
                const Param q = param_of(ro_lds[bcast ? 0u : l * units + u]);
                r[l] = rope_elem(x[l], lo ? -(i64)p[l] : (i64)p[l], cs[l], sn[l], q);
            }
        } else {
            int y[8];
            ld_unit<0>(rb, u, y);
#pragma unroll
            for (int l = 0; l < 8; l++) {
                const Param q = param_of(ro_lds[bcast ? 0u : l * units + u]);
                if constexpr (CODE == RO_MULACT) {
                    r[l] = mulact_elem(x[l], y[l], q, tab);
                } else {   // GATE
                    if (q.sa <= 23 && q.sb <= 23 && q.sc <= 61) {
                        const i64 th = 2 * sig_q((i64)x[l] << q.sa, tab) - ((i64)1 << 24);
                        const i64 sg = sig_q((i64)y[l] << q.sb, tab);
                        r[l] = (int)sat16(rne_shr_fast(th * sg, (uint32_t)q.sc));
                    } else {
                        const i64 th = 2 * sig_q((i64)x[l] << q.sa, tab) - ((i64)1 << 24);
                        const i64 sg = sig_q((i64)y[l] << q.sb, tab);
                        r[l] = (int)sat16(rne_shr((i128)th * sg, q.sc));
                    }
                }
            }
        }
        store_stream(rc + 16u * u, pack16(r));
    }
}

// ---------------------------------------------------------------- TRANSPOSE
// tile (i2, i1): R rows (b_s1 apart) of L = n int16; column d -> granule at c + d * b_s2.
__global__ __launch_bounds__(256) void ro_xpose_kernel(Job j) {
    const uint32_t R = j.aux & 15, L = j.n;
    const u64 total = (u64)L * R * j.c1 * j.c2;
    for (u64 e = (u64)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (u64)gridDim.x * blockDim.x) {
        const uint32_t r = (uint32_t)(e % R);
        const u64 t1 = e / R;
        const uint32_t d = (uint32_t)(t1 % L);
        const u64 tile = t1 / L;
        const uint32_t i1 = (uint32_t)(tile % j.c1), i2 = (uint32_t)(tile / j.c1);
        const uint8_t* ta = j.a + (u64)i2 * j.a_s2 + (u64)i1 * j.a_s1;
        uint8_t* tc = j.c + (u64)i2 * j.c_s2 + (u64)i1 * j.c_s1;
        *reinterpret_cast<int16_t*>(tc + (u64)d * j.b_s2 + 2u * r) =
            *reinterpret_cast<const int16_t*>(ta + (u64)r * j.b_s1 + 2u * d);
        // a contiguous tile ends on a whole word: the lanes past L * R are zero
        if (j.b_s2 == 2 * R && d == L - 1 && r == R - 1)
            for (u64 o = 2ull * R * L; o % 16; o += 2) *reinterpret_cast<int16_t*>(tc + o) = 0;
    }
}

// ---------------------------------------------------------------- FOLD
// rne(x / (m_x 2^s)), m_x = m for x < 0, 1 otherwise (rowops_spec.fold_elem)
__device__ __forceinline__ i64 fold_elem(i64 x, uint32_t m, uint32_t s) {
    const i64 u = x < 0 ? -x : x, den = (i64)(x < 0 ? m : 1u) << s;
    i64 q = u / den;
    const i64 r = u - q * den;
    q += (2 * r > den || (2 * r == den && (q & 1))) ? 1 : 0;
    return x < 0 ? -q : q;
}

__global__ __launch_bounds__(256) void ro_fold_kernel(Job j) {
    const uint32_t s = j.aux & 15, m = (j.aux >> 4) & 127;
    const u64 total = (u64)j.c2 * j.c1 * j.n;
    const u64 padded = (total + 7) & ~7ull;
    for (u64 o = (u64)blockIdx.x * blockDim.x + threadIdx.x; o < padded; o += (u64)gridDim.x * blockDim.x) {
        i64 v = 0;
        if (o < total) {
            const uint32_t col = (uint32_t)(o % j.n);
            const u64 t1 = o / j.n;
            const uint32_t r = (uint32_t)(t1 % j.c1);
            const u64 k = t1 / j.c1;
            const i64 src = (i64)(int32_t)j.b_s2 + (i64)r * j.b_s1 + (i64)col;
            if (src >= (i64)j.win_lo && src < (i64)j.win_hi)
                v = fold_elem(*reinterpret_cast<const int16_t*>(j.a + (i64)k * (int32_t)j.a_s2 + 2 * src), m, s);
        }
        *reinterpret_cast<int16_t*>(j.c + 2 * o) = (int16_t)v;
    }
}

// ---------------------------------------------------------------- TLOAD
// The table image as rows of int32 delivered in order (c2 blocks of c1 rows of n words).
__global__ __launch_bounds__(256) void ro_tload_kernel(Job j, uint8_t* __restrict__ tab) {
    const u64 total = (u64)j.n * j.c1 * j.c2;
    for (u64 e = (u64)blockIdx.x * blockDim.x + threadIdx.x; e < total && e < 16384;
         e += (u64)gridDim.x * blockDim.x) {
        const uint32_t col = (uint32_t)(e % j.n);
        const u64 row = e / j.n;
        const uint32_t i1 = (uint32_t)(row % j.c1), i2 = (uint32_t)(row / j.c1);
        *reinterpret_cast<uint32_t*>(tab + 4 * e) =
            *reinterpret_cast<const uint32_t*>(j.a + (u64)i2 * j.a_s2 + (u64)i1 * j.a_s1 + 4u * col);
    }
}

// ---------------------------------------------------------------- decode prep
// A decode step's attention prep in one launch: q and k rows [B][heads HD] RoPE'd at one
// position (the ROPE jobs of the two RopeRoNodes: their parameter blocks, the table row of the
// position), q into qr, k straight into the K cache rows kc[b][g][pos] and v copied into the V
// cache rows vc[b][g][pos] (caches [B][KV][C][HD]): the ROPE, ROPE and the two KV row writes of
// the unfused step, with the same element rule (rope_value).  A thread per 16-byte output word.
struct DecodePrep {
    const int16_t *q, *k, *v;
    int16_t *qr, *kc, *vc;
    const int32_t* tab;                 // cos [HD] then sin [HD] of the position
    const uint8_t *pq, *pk;             // the ROPE jobs' parameter blocks
    uint32_t bcq, bck, B, H, KV, HD, C, pos;
};

__global__ __launch_bounds__(256) void decode_prep_kernel(DecodePrep d) {
    const uint32_t qw = d.H * d.HD / 8, kw = d.KV * d.HD / 8, per = qw + 2 * kw;
    const u64 total = (u64)d.B * per;
    for (u64 w = (u64)blockIdx.x * blockDim.x + threadIdx.x; w < total; w += (u64)gridDim.x * blockDim.x) {
        const uint32_t b = (uint32_t)(w / per), r = (uint32_t)(w - (u64)b * per);
        int16_t* dst;
        uint32_t out[4] = {0, 0, 0, 0};
        if (r < qw + kw) {
            const bool isq = r < qw;
            const uint32_t col0 = (isq ? r : r - qw) * 8, d0 = col0 % d.HD;
            const int16_t* row = isq ? d.q + (u64)b * d.H * d.HD : d.k + (u64)b * d.KV * d.HD;
            const uint8_t* prm = isq ? d.pq : d.pk;
            const bool bc = (isq ? d.bcq : d.bck) != 0;
            const int4 xw = *reinterpret_cast<const int4*>(row + col0);
            const int4 pw = *reinterpret_cast<const int4*>(row + (d0 < d.HD / 2 ? col0 + d.HD / 2 : col0 - d.HD / 2));
            const uint4 o = rope_unit8(xw, pw, d.tab, d.HD, d0, [&](uint32_t l) { return ld_param(prm, col0 + l, bc); });
            out[0] = o.x; out[1] = o.y; out[2] = o.z; out[3] = o.w;
            dst = isq ? d.qr + (u64)b * d.H * d.HD + col0
                      : d.kc + (((u64)b * d.KV + col0 / d.HD) * d.C + d.pos) * d.HD + col0 % d.HD;
        } else {
            const uint32_t col0 = (r - qw - kw) * 8;
            const uint4 x = *reinterpret_cast<const uint4*>(d.v + (u64)b * d.KV * d.HD + col0);
            out[0] = x.x; out[1] = x.y; out[2] = x.z; out[3] = x.w;
            dst = d.vc + (((u64)b * d.KV + col0 / d.HD) * d.C + d.pos) * d.HD + col0 % d.HD;
        }
        *reinterpret_cast<uint4*>(dst) = make_uint4(out[0], out[1], out[2], out[3]);
    }
}

unsigned grid_for(u64 items, unsigned per_block = 256) {
    u64 b = (items + per_block - 1) / per_block;
    if (b > 65536ull * 8) b = 65536ull * 8;
    return (unsigned)(b ? b : 1);
}

bool norm_fast_ok(const Job& j) {
    const uint32_t ak = (j.op >> 4) & 3;
    const bool a_words = aligned16(j.a) && (j.a_s1 & 15) == 0 && (j.a_s2 & 15) == 0;
    return (j.n & 7) == 0 && a_words && ak <= 1 && j.bq_sh <= 40;
}

// The fast NORM of job j (norm_fast_ok), after the ADDX job `ja` with parameters pa (ADDX),
// writing the byte planes `po` of its output (PL).
int run_norm_fast(DeviceState* st, const Job& j, const uint8_t* params, uint8_t* dst, uint32_t entries, bool bcast,
                  const Job* ja, const uint8_t* pa, bool bca, const APlanes* po, hipStream_t s) {
    const uint32_t units = j.n / 8;
    const uint32_t upl = units <= 64 ? 1 : 2;        // larger rows take the workgroup kernel above
    // with the ADDX job two parameter blocks are staged per workgroup: fewer workgroups, more
    // rows each (measured at BERT's 3072 x 768: 17.3 us at two per CU, 19.2 at eight)
    const unsigned blocks = (unsigned)std::min<u64>(((u64)j.c1 * j.c2 + 3) / 4, (u64)st->cus * (ja != nullptr ? 2 : 8));
    // two units a lane and at least twelve rows per CU: one workgroup of twelve wavefronts per
    // CU (three a SIMD, the most the registers allow), a row per wavefront at a time, so that a
    // CU stages the parameter blocks once and issues all its rows' loads at the start
    // (BERT's 3072 x 768 ADDX + LayerNorm with planes: 14.6 -> 13.8 us, the LayerNorm with
    // planes 9.4 -> 8.8 us)
    const bool wide_wg = upl == 2 && (u64)j.c1 * j.c2 >= (u64)st->cus * 12;
    const size_t plds = (size_t)((bcast ? 1 : j.n) + (ja != nullptr ? (bca ? 1 : ja->n) : 0)) * 16;
    const uint32_t ak = ja != nullptr ? (ja->op >> 4) & 3 : (j.op >> 4) & 3;
    const Job jx = ja != nullptr ? *ja : j;
    const APlanes pv = po != nullptr ? *po : APlanes{};
    const uint32_t sel = (ak ? 1u : 0u) | (ja != nullptr ? 2u : 0u) | (po != nullptr ? 4u : 0u);
    const u64 rows = (u64)j.c1 * j.c2;
    if ((rows <= (u64)st->cus || units > 128) && units <= 512) {
        // rows that do not fill the chip (the decode step's 16), or rows past 1024 elements
        // (four or more units a lane would spill): a workgroup of 256 per row, rows in turn over
        // at most four workgroups per CU so that each stages the parameters once for many rows
        const unsigned wblocks = (unsigned)std::min<u64>(rows, (u64)st->cus * 4);
#define CM_NORM_WG(AK, U, AX, PL, T)                                                                                \
    CM_LAUNCH("ro_norm_kernel", (ro_norm_wg_kernel<AK, U, AX, PL, T>), dim3(wblocks), dim3(T), plds, s, j, params,  \
              dst, entries, bcast, st->ro_tables, jx, pa, bca, pv)
#define CM_NORM_WG_T(AK, AX, PL)                                                                                    \
    if (units <= 256) { CM_NORM_WG(AK, 1, AX, PL, 256); } else { CM_NORM_WG(AK, 2, AX, PL, 256); }
        switch (sel) {
        case 0: { CM_NORM_WG_T(0, false, false) } break;
        case 1: { CM_NORM_WG_T(1, false, false) } break;
        case 4: { CM_NORM_WG_T(0, false, true) } break;
        case 5: { CM_NORM_WG_T(1, false, true) } break;
        case 2: { CM_NORM_WG_T(0, true, false) } break;
        case 3: { CM_NORM_WG_T(1, true, false) } break;
        case 6: { CM_NORM_WG_T(0, true, true) } break;
        default: { CM_NORM_WG_T(1, true, true) } break;
        }
#undef CM_NORM_WG_T
#undef CM_NORM_WG
        return CM_OK;
    }
#define CM_NORM(AK, U, AX, PL, NW, B)                                                                              \
    CM_LAUNCH("ro_norm_kernel", (ro_norm_fast_kernel<AK, U, AX, PL, NW>), dim3(B), dim3(64 * NW), plds, s, j, params, \
              dst, entries, bcast, st->ro_tables, jx, pa, bca, pv)
#define CM_NORM_U(AK, AX, PL)                                                                                      \
    if (upl == 1) { CM_NORM(AK, 1, AX, PL, 4, blocks); }                                                            \
    else if (wide_wg) { CM_NORM(AK, 2, AX, PL, 12, st->cus); }                                                      \
    else { CM_NORM(AK, 2, AX, PL, 4, blocks); }
    switch (sel) {
    case 0: { CM_NORM_U(0, false, false) } break;
    case 1: { CM_NORM_U(1, false, false) } break;
    case 4: { CM_NORM_U(0, false, true) } break;
    case 5: { CM_NORM_U(1, false, true) } break;
    case 2: { CM_NORM_U(0, true, false) } break;
    case 3: { CM_NORM_U(1, true, false) } break;
    case 6: { CM_NORM_U(0, true, true) } break;
    default: { CM_NORM_U(1, true, true) } break;
    }
#undef CM_NORM_U
#undef CM_NORM
    return CM_OK;
}

int run_job(DeviceState* st, const Job& j, const uint8_t* p, hipStream_t s) {
    const uint32_t code = j.op & 15;
    if (code == RO_TLOAD) {
        if (j.n == 0 || j.c1 == 0 || j.c2 == 0) return CM_OK;
        CM_LAUNCH("ro_tload_kernel", ro_tload_kernel, dim3(grid_for((u64)j.n * j.c1 * j.c2)), dim3(256), 0, s, j,
                           st->ro_tables);
        return CM_OK;
    }
    if (code == RO_FOLD) {
        const uint32_t m = (j.aux >> 4) & 127;
        if (j.n == 0 || j.c1 == 0 || j.c2 == 0 || m == 0) return CM_OK;
        if (j.c == nullptr) return fail(CM_EINVAL, "rowops FOLD: a null output");
        if (reinterpret_cast<uintptr_t>(j.c) & 15) return fail(CM_EALIGN, "rowops FOLD: c not 16-byte aligned");
        const u64 total = ((u64)j.c2 * j.c1 * j.n + 7) & ~7ull;
        CM_LAUNCH("ro_fold_kernel", ro_fold_kernel, dim3(grid_for(total)), dim3(256), 0, s, j);
        return CM_OK;
    }
    if (j.n == 0 || j.c1 == 0 || j.c2 == 0) return CM_OK;
    if (j.n > kNMax) return fail(CM_EINVAL, "rowops: n = %u above %u", j.n, kNMax);
    if (code == RO_XPOSE) {
        const uint32_t R = j.aux & 15;
        if (R == 0 || R > 8) return CM_OK;        // outside the contract: the unit writes nothing
        if (j.c == nullptr) return fail(CM_EINVAL, "rowops TRANSPOSE: a null output");
        CM_LAUNCH("ro_xpose_kernel", ro_xpose_kernel, dim3(grid_for((u64)j.n * R * j.c1 * j.c2)), dim3(256), 0, s, j);
        return CM_OK;
    }
    if (code < RO_COPY || code > RO_GATE) return fail(CM_EINVAL, "rowops: op code %u", code);
    if (code == RO_ROPE) {
        const uint32_t HD = j.aux & 0xFFF;
        if (HD == 0 || (HD & 15) || HD > 128 || j.n % HD) return CM_OK;   // the unit writes nothing
    }
    // every job here writes c: a null output is refused (only cm_rowops_chain_planes' last NORM,
    // whose rows its planes replace, may have none, and that job does not come through here)
    if (j.c == nullptr) return fail(CM_EINVAL, "rowops: a null output");
    if ((reinterpret_cast<uintptr_t>(j.c) & 15) || (j.c_s1 & 15) || (j.c_s2 & 15))
        return fail(CM_EALIGN, "rowops: c and its strides must be 16-byte aligned");
    // parameter RAM: a load (unless P_KEEP finds a valid RAM) or the RAM as the last load left it
    const bool keep = (j.op & F_P_KEEP) && st->pram_valid;
    const bool bcast_job = (j.op & F_P_BCAST) != 0;
    const uint8_t* params;
    uint8_t* dst = nullptr;
    uint32_t entries = 0;
    bool bcast;
    if (keep) {
        params = st->ro_pram;
        bcast = st->pram_bcast;
    } else {
        if (p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15)) return fail(CM_EALIGN, "rowops: p must be 16-byte aligned");
        params = p;
        bcast = bcast_job;
        dst = st->ro_pram;
        entries = bcast_job ? 1 : j.n;
        st->pram_valid = true;
        st->pram_bcast = bcast_job;
    }
    const uint32_t ak = (j.op >> 4) & 3, bk = (j.op >> 6) & 3, ck = (j.op >> 8) & 3;
    const bool a_words = aligned16(j.a) && (j.a_s1 & 15) == 0 && (j.a_s2 & 15) == 0;
    const bool b_words = aligned16(j.b) && (j.b_s1 & 15) == 0 && (j.b_s2 & 15) == 0;
    const size_t plds = (size_t)(bcast ? 1 : j.n) * 16;
    if (code == RO_NORM) {
        if (norm_fast_ok(j)) return run_norm_fast(st, j, params, dst, entries, bcast, nullptr, nullptr, false, nullptr, s);
        CM_LAUNCH("ro_norm_kernel", ro_norm_kernel, dim3(grid_for((u64)j.c1 * j.c2, 4)), dim3(256), 0, s, j, params,
                           dst, entries, bcast, st->ro_tables);
        return CM_OK;
    }
    const bool ben = (j.op & F_B_EN) != 0;
    if ((code == RO_COPY || code == RO_ADDX) && (j.n & 7) == 0 && a_words && (!ben || b_words) && ak <= 1 &&
        bk <= 1 && ck <= 1) {
        const u64 units = (u64)(j.n / 8) * j.c1 * j.c2;
        const unsigned blocks = (unsigned)std::min<u64>((units + 255) / 256, (u64)st->cus * 16);
        const uint32_t sel = ak | (bk << 1) | (ck << 2) | ((ben ? 1u : 0u) << 3);
#define CM_ADDX(AK, BK, CK, BEN)                                                                                   \
    case AK | (BK << 1) | (CK << 2) | (BEN << 3):                                                                 \
        CM_LAUNCH("ro_stream_kernel", (ro_addx_fast_kernel<AK, BK, CK, BEN != 0>), dim3(blocks), dim3(256), plds, s, \
                  j, params, dst, entries, bcast);                                                                 \
        return CM_OK;
        switch (sel) {
            CM_ADDX(0, 0, 0, 0) CM_ADDX(1, 0, 0, 0) CM_ADDX(0, 1, 0, 0) CM_ADDX(1, 1, 0, 0)
            CM_ADDX(0, 0, 1, 0) CM_ADDX(1, 0, 1, 0) CM_ADDX(0, 1, 1, 0) CM_ADDX(1, 1, 1, 0)
            CM_ADDX(0, 0, 0, 1) CM_ADDX(1, 0, 0, 1) CM_ADDX(0, 1, 0, 1) CM_ADDX(1, 1, 0, 1)
            CM_ADDX(0, 0, 1, 1) CM_ADDX(1, 0, 1, 1) CM_ADDX(0, 1, 1, 1) CM_ADDX(1, 1, 1, 1)
        default: break;
        }
#undef CM_ADDX
    }
    const bool c_words = aligned16(j.c) && (j.c_s1 & 15) == 0 && (j.c_s2 & 15) == 0;
    if ((code == RO_DEQUANT || code == RO_MULACT || code == RO_GATE || code == RO_ROPE) && (j.n & 7) == 0 &&
        a_words && c_words && ak == 0 && (code == RO_DEQUANT || ck == 0) &&
        (code == RO_DEQUANT || (b_words && (code == RO_ROPE || (bk == 0 && ben))))) {
        const u64 units = (u64)(j.n / 8) * j.c1 * j.c2;
        const unsigned blocks = (unsigned)std::min<u64>((units + 255) / 256, (u64)st->cus * 16);
#define CM_UNIT(C)                                                                                                   \
    CM_LAUNCH("ro_stream_kernel", ro_unit_fast_kernel<C>, dim3(blocks), dim3(256), plds, s, j, params, dst, entries, \
              bcast, st->ro_tables);                                                                                 \
    return CM_OK;
        if (code == RO_DEQUANT) { CM_UNIT(RO_DEQUANT) }
        if (code == RO_MULACT) { CM_UNIT(RO_MULACT) }
        if (code == RO_GATE) { CM_UNIT(RO_GATE) }
        CM_UNIT(RO_ROPE)
#undef CM_UNIT
    }
    const uint32_t cb = code == RO_DEQUANT ? 4 : (((j.op >> 8) & 3) == 0 ? 2 : 4);
    const u64 words = (u64)((j.n * cb + 15) / 16) * j.c1 * j.c2;
    CM_LAUNCH("ro_stream_kernel", ro_stream_kernel, dim3(grid_for(words)), dim3(256), 0, s, j, params, dst, entries,
                       bcast, st->ro_tables);
    return CM_OK;
}

}  // namespace
}  // namespace cm

extern "C" int cm_rowops(const void* a, const void* b, void* c, const void* p, uint32_t op,
                         uint32_t n, uint32_t c1, uint32_t c2, uint32_t a_s1, uint32_t a_s2,
                         uint32_t b_s1, uint32_t b_s2, uint32_t c_s1, uint32_t c_s2, int64_t eps,
                         uint32_t aux, uint32_t bq_sh, uint32_t win_lo, uint32_t win_hi, void* stream) {
    using namespace cm;
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    Job j{static_cast<const uint8_t*>(a), static_cast<const uint8_t*>(b), static_cast<uint8_t*>(c), op, n, c1,
          c2, a_s1, a_s2, b_s1, b_s2, c_s1, c_s2, eps, aux, bq_sh, win_lo, win_hi};
    return run_job(st, j, static_cast<const uint8_t*>(p), as_stream(stream));
}

namespace cm {
namespace {

Job job_of(const cm_rowops_desc& d) {
    return Job{reinterpret_cast<const uint8_t*>(d.a), reinterpret_cast<const uint8_t*>(d.b),
               reinterpret_cast<uint8_t*>(d.c), d.op, d.n, d.c1, d.c2, d.a_s1, d.a_s2, d.b_s1, d.b_s2, d.c_s1, d.c_s2,
               d.eps, d.aux, d.bq_sh, d.win_lo, d.win_hi};
}

// The jobs' own parameter block, 16-byte aligned (P_KEEP jobs are not fused).
bool own_params(const cm_rowops_desc& d) {
    return !(d.op & F_P_KEEP) && d.p != 0 && (d.p & 15) == 0;
}

// Job b is a fast NORM of job a's int32 output over the same rows, and a is a COPY / ADDX of
// whole 8-element units (int32 or int16 A, int16 B, no window): the pair runs as one launch.
bool fusable_addx_norm(const cm_rowops_desc& a, const cm_rowops_desc& b) {
    const uint32_t code = a.op & 15, ak = (a.op >> 4) & 3, bk = (a.op >> 6) & 3, ck = (a.op >> 8) & 3;
    if ((code != RO_ADDX && code != RO_COPY) || !(a.op & F_B_EN) || ak > 1 || bk != 0 || ck != 1) return false;
    if ((b.op & 15) != RO_NORM || ((b.op >> 4) & 3) != 1 || !own_params(a) || !own_params(b)) return false;
    if (a.n != b.n || a.c1 != b.c1 || a.c2 != b.c2 || a.n == 0 || (a.n & 7) || a.n > 4096) return false;
    if (b.a != a.c || b.a_s1 != a.c_s1 || b.a_s2 != a.c_s2 || a.win_lo != 0 || a.win_hi < a.c1) return false;
    // both parameter blocks staged in the default 64 KiB of dynamic LDS
    const size_t plds = 16 * (size_t)(((a.op & F_P_BCAST) ? 1 : a.n) + ((b.op & F_P_BCAST) ? 1 : b.n));
    if (plds > 65536) return false;
    const bool words = (a.a & 15) == 0 && (a.b & 15) == 0 && (a.c & 15) == 0 && (b.c & 15) == 0 &&
                       ((a.a_s1 | a.a_s2 | a.b_s1 | a.b_s2 | a.c_s1 | a.c_s2 | b.c_s1 | b.c_s2) & 15) == 0;
    return words && norm_fast_ok(job_of(b));
}

int run_chain(const cm_rowops_desc* jobs, uint32_t n_jobs, void* planes, hipStream_t s) {
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    if (planes != nullptr) {
        if (n_jobs == 0) return fail(CM_EINVAL, "rowops chain: planes of no job");
        const cm_rowops_desc& l = jobs[n_jobs - 1];
        if ((l.op & 15) != RO_NORM || ((l.op >> 8) & 3) != 0 || (l.n % 64) || l.n > 4096 || !own_params(l) ||
            !norm_fast_ok(job_of(l)) || (l.c & 15) || ((l.c_s1 | l.c_s2) & 15) ||
            (reinterpret_cast<uintptr_t>(planes) & 255))
            return fail(CM_EINVAL, "rowops chain: planes need a last NORM job of int16 rows of a multiple of 64 "
                                   "(its own parameters, 256-byte aligned planes)");
    }
    for (uint32_t i = 0; i < n_jobs; i++) {
        const bool last = i + 1 == n_jobs;
        const bool fuse = i + 1 < n_jobs && fusable_addx_norm(jobs[i], jobs[i + 1]);
        const bool pl = planes != nullptr && (last || (fuse && i + 2 == n_jobs));
        if (!fuse && !pl) {
            const cm_rowops_desc& d = jobs[i];
            rc = cm_rowops(reinterpret_cast<const void*>(d.a), reinterpret_cast<const void*>(d.b),
                           reinterpret_cast<void*>(d.c), reinterpret_cast<const void*>(d.p), d.op, d.n, d.c1, d.c2,
                           d.a_s1, d.a_s2, d.b_s1, d.b_s2, d.c_s1, d.c_s2, d.eps, d.aux, d.bq_sh, d.win_lo, d.win_hi,
                           s);
            if (rc) return rc;
            continue;
        }
        const cm_rowops_desc& dn = jobs[fuse ? i + 1 : i];
        // the NORM's rows may stay unwritten only when this launch writes their planes (the
        // chain's last job); the residual sum of a fused ADDX is always written
        if ((dn.c == 0 && !pl) || (fuse && jobs[i].c == 0))
            return fail(CM_EINVAL, "rowops chain: a null output (only the planes' NORM may leave its rows unwritten)");
        const Job jn = job_of(dn);
        if (jn.c1 == 0 || jn.c2 == 0) {
            i += fuse ? 1 : 0;
            continue;
        }
        Job ja{};
        const uint8_t* pa = nullptr;
        bool bca = false;
        if (fuse) {
            ja = job_of(jobs[i]);
            pa = reinterpret_cast<const uint8_t*>(jobs[i].p);
            bca = (jobs[i].op & F_P_BCAST) != 0;
        }
        const bool bcn = (dn.op & F_P_BCAST) != 0;
        st->pram_valid = true;           // the NORM's block is the one the RAM keeps
        st->pram_bcast = bcn;
        APlanes pv{};
        if (pl) {
            const uint32_t rows = jn.c1 * jn.c2;
            pv = a_planes_view(planes, rows, jn.n, (jn.n + 1023) / 1024);
        }
        rc = run_norm_fast(st, jn, reinterpret_cast<const uint8_t*>(dn.p), st->ro_pram, bcn ? 1u : jn.n, bcn,
                           fuse ? &ja : nullptr, pa, bca, pl ? &pv : nullptr, s);
        if (rc) return rc;
        i += fuse ? 1 : 0;
    }
    return CM_OK;
}

}  // namespace
}  // namespace cm

extern "C" int cm_rowops_chain(const cm_rowops_desc* jobs, uint32_t n_jobs, void* stream) {
    return cm::run_chain(jobs, n_jobs, nullptr, cm::as_stream(stream));
}

extern "C" int cm_rowops_chain_planes(const cm_rowops_desc* jobs, uint32_t n_jobs, void* planes, void* stream) {
    if (planes == nullptr) return cm::fail(CM_EINVAL, "rowops chain: no planes buffer");
    return cm::run_chain(jobs, n_jobs, planes, cm::as_stream(stream));
}

extern "C" int cm_decode_prep(const int16_t* q, const int16_t* k, const int16_t* v, int16_t* qr, int16_t* kc,
                              int16_t* vc, uint32_t batch, uint32_t heads, uint32_t kv_heads, uint32_t head_dim,
                              uint32_t cache_rows, uint32_t pos, const void* rope_row, const void* params_q,
                              uint32_t op_q, const void* params_k, uint32_t op_k, void* stream) {
    using namespace cm;
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    if (batch == 0) return CM_OK;
    if (head_dim == 0 || (head_dim & 15) || head_dim > 128 || heads == 0 || kv_heads == 0)
        return fail(CM_EINVAL, "decode prep: %u heads and %u KV heads of %u (a multiple of 16 up to 128)", heads,
                    kv_heads, head_dim);
    if (pos >= cache_rows) return fail(CM_EINVAL, "decode prep: position %u of %u cache rows", pos, cache_rows);
    for (uint32_t op : {op_q, op_k})
        if ((op & 15) != RO_ROPE || ((op >> 4) & 3) != 0 || ((op >> 8) & 3) != 0 || (op & F_P_KEEP))
            return fail(CM_EINVAL, "decode prep: 0x%x is not an int16 ROPE job's op word", op);
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(qr) || !aligned16(kc) || !aligned16(vc) ||
        !aligned16(rope_row) || (reinterpret_cast<uintptr_t>(params_q) & 15) ||
        (reinterpret_cast<uintptr_t>(params_k) & 15))
        return fail(CM_EALIGN, "decode prep: operands not aligned");
    const DecodePrep d{q, k, v, qr, kc, vc, static_cast<const int32_t*>(rope_row),
                       static_cast<const uint8_t*>(params_q), static_cast<const uint8_t*>(params_k),
                       (op_q & F_P_BCAST) ? 1u : 0u, (op_k & F_P_BCAST) ? 1u : 0u, batch, heads, kv_heads, head_dim,
                       cache_rows, pos};
    const uint64_t words = (uint64_t)batch * (heads + 2 * kv_heads) * head_dim / 8;
    CM_LAUNCH("decode_prep_kernel", decode_prep_kernel, dim3(grid_for(words)), dim3(256), 0, as_stream(stream), d);
    return CM_OK;
}
