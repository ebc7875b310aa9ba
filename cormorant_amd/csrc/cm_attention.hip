// cm_attention.hip -- the attention block of an encoder layer in one kernel: per (sequence,
// head) and block of 64 queries,
//   s[j][i] = sat16(wrap32(sum_d K[j][d] Q[i][d]) >> 8)          (q.K^T, keys-major)
//   P[i][.] = the softmax unit's column mode over the keys of query i (all keys valid)
//   o[i][d] = sat16(wrap32(sum_j P[i][j] V[j][d]) >> 8)          (P.V)
// with Q, K, V read straight from the fused projection's rows and o written into the merged
// token-major rows: the chain of the reference's VitAttnPrep, the q.K^T contraction, the
// VitAttnSoftmax keys-major call, the P.V contraction and the head merge (vit.py:19-32,
// llm_nodes.py:995-1001, vectorop_smx.py:50-66), without materializing s or P.
//
// Both contractions run on v_mfma_i32_16x16x64_i8 over byte limbs: x - 128 = 256 h + l with
// h = x >> 8 and l = (x & 255) - 128, so that
//   sum a b = 2^16 HH + 2^8 (HL + LH) + LL + 128 sum a + 128 sum b - 16384 K   (mod 2^32),
// the int32-wrapped sum exactly (the wrap makes every term's order free).  Phase 1 takes the
// operand sums as limb sums from MFMAs against an all-ones operand, already in the result
// layout; phase 3 takes them from the staging and a lane-group reduction.
//
// Workgroup: 4 wavefronts, wavefront w owns queries q0 + 16 w .. + 15 end to end.  MFMA
// layouts (16 x 16 blocks): operand lane l holds row / column l % 16 and 16 bytes of k slot
// group l / 16; result lane l holds column l % 16, rows 4 (l / 16) .. + 3.
//   phase 1: s for key block kb (16 keys) = K rows (A: from the projection rows, split into
//            limbs once per workgroup, 64 keys at a time through LDS) x Q rows (B, loaded once): lane (query l % 16, g = l / 16) ends up
//            with the scores of keys 16 kb + 4 g + r, r < 4, for all T / 16 blocks;
//   phase 2: the softmax per query over its lane group (shuffles across g; no LDS):
//            e = TAB[y & 4095] >> (y >> 12), y = (max - s) Cm >> Cs, R = floor(2^40 / S),
//            P = min((e R + 2^(39 - fp)) >> (40 - fp), 32767) (the unit's integer rule; y in
//            32 bits below dlim, P through an exact double);
//   phase 3: o^T = V^T P^T: P stays in registers as the B operand, its k slots the lane's own
//            keys (slot 16 g + 4 q + r of k step ks = key 16 (4 ks + q) + 4 g + r); V^T is
//            split into byte planes in LDS in that key order, 32 d at a time (the first half
//            staged before phase 1, the second after the first half's products).
// LDS: TAB (16 KiB; during phase 1 the K chunks' limbs, two buffers of 64 keys) + V^T hi / lo
// planes [32][T + 16] + the V column-sum partials, 42.6 KiB at T = 384: three workgroups per
// compute unit, so that BERT's 576 workgroups are resident at once.
#include "cm_common.h"

#include <algorithm>

namespace cm {
namespace {

constexpr uint32_t kHd = 64;                 // head dimension
constexpr uint32_t kQb = 64;                 // queries per workgroup

typedef int v4i __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int sat16_shr8(int acc) { return min(max(acc >> 8, -32768), 32767); }

// 8 int16 -> their high bytes and low bytes ^ 0x80 (two dwords each)
__device__ __forceinline__ void limbs8(const int4 v, uint32_t& h0, uint32_t& h1, uint32_t& l0, uint32_t& l1) {
    const uint32_t x = (uint32_t)v.x, y = (uint32_t)v.y, z = (uint32_t)v.z, u = (uint32_t)v.w;
    h0 = __builtin_amdgcn_perm(y, x, 0x07050301u);
    h1 = __builtin_amdgcn_perm(u, z, 0x07050301u);
    l0 = __builtin_amdgcn_perm(y, x, 0x06040200u) ^ 0x80808080u;
    l1 = __builtin_amdgcn_perm(u, z, 0x06040200u) ^ 0x80808080u;
}

// 16 consecutive int16 at p (16-byte aligned) -> the hi / lo limb operands
__device__ __forceinline__ void limbs16(const int16_t* p, v4i& hi, v4i& lo) {
    const int4 a = *reinterpret_cast<const int4*>(p), b = *reinterpret_cast<const int4*>(p + 8);
    uint32_t h0, h1, h2, h3, l0, l1, l2, l3;
    limbs8(a, h0, h1, l0, l1);
    limbs8(b, h2, h3, l2, l3);
    hi = v4i{(int)h0, (int)h1, (int)h2, (int)h3};
    lo = v4i{(int)l0, (int)l1, (int)l2, (int)l3};
}

__device__ __forceinline__ uint32_t dword(const int4& v, uint32_t q) {
    return (uint32_t)(q == 0 ? v.x : q == 1 ? v.y : q == 2 ? v.z : v.w);
}

__device__ __forceinline__ v4i mfma(v4i a, v4i b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// the wrapped sum from the limb accumulators and the row + column term 128 (ra + cb) - 16384 K
__device__ __forceinline__ int32_t wrap_sum(int32_t hh, int32_t mid, int32_t ll, uint32_t term) {
    return (int32_t)(((uint32_t)hh << 16) + ((uint32_t)mid << 8) + (uint32_t)ll + term);
}

// T = keys per sequence (a multiple of 64, at most 384).  qkv rows: ld elements apart; Q / K /
// V of head h at columns q_off / k_off / v_off + 64 h.  o rows: o_ld apart, head h at 64 h.
// PL: also the byte planes of o as the A operand of the output projection (rows b T + i, the
// row sums of head h's 64 columns as partial sum h).
template <uint32_t T, bool PL>
__global__ __launch_bounds__(256, 3) void attention_kernel(const int16_t* __restrict__ qkv, int16_t* __restrict__ o,
                                                           const int32_t* __restrict__ tab, uint32_t heads,
                                                           uint64_t ld, uint32_t q_off, uint32_t k_off,
                                                           uint32_t v_off, uint64_t o_ld, uint32_t cm, uint32_t cfg,
                                                           uint32_t dlim, APlanes po) {
    constexpr uint32_t KB = T / 16;          // key blocks of phase 1
    constexpr uint32_t KS = T / 64;          // k steps of phase 3
    constexpr uint32_t VS = T + 16;          // V^T plane row stride, bytes (rows 4 banks apart)
    constexpr uint32_t HD = kHd / 2;         // d per staged half
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    int32_t* stab = reinterpret_cast<int32_t*>(lds);                      // [4096]
    uint8_t* vth = lds + 16384;                                           // [32][VS]
    uint8_t* vtl = vth + HD * VS;                                         // [32][VS]
    int32_t* vsw = reinterpret_cast<int32_t*>(vtl + HD * VS);             // [4][64]

    const uint32_t t = threadIdx.x, lane = t & 63, w = t >> 6, c16 = lane & 15, g = lane >> 4;
    const uint32_t bh = blockIdx.y, b = bh / heads, h = bh - b * heads;
    const uint32_t q0 = blockIdx.x * kQb;
    const int16_t* seq = qkv + (uint64_t)b * T * ld;

    // V^T planes of d 32 half .. + 31 (task = 4 keys x 8 d: keys 4 qd + r, d 8 (4 half + c) ..)
    // and the per-wavefront column sums of those d
    auto stage_v = [&](uint32_t half) {
        const uint32_t c = t & 3;
        int vpart[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (uint32_t it = 0; it < (T / 4 + 63) / 64; it++) {
            const uint32_t qd = (t >> 2) + 64 * it;
            if (qd >= T / 4) break;
            const int16_t* vp = seq + (uint64_t)(4 * qd) * ld + v_off + kHd * h + HD * half + 8 * c;
            int4 x[4];
#pragma unroll
            for (uint32_t r = 0; r < 4; r++) x[r] = *reinterpret_cast<const int4*>(vp + (uint64_t)r * ld);
            // key 16 kb + 4 g' + r sits at position 64 (kb / 4) + 16 g' + 4 (kb % 4) + r
            const uint32_t p0 = 64 * (qd >> 4) + 16 * (qd & 3) + 4 * ((qd >> 2) & 3);
#pragma unroll
            for (uint32_t q = 0; q < 4; q++) {
                const uint32_t a0 = dword(x[0], q), a1 = dword(x[1], q), a2 = dword(x[2], q), a3 = dword(x[3], q);
                const uint32_t th01 = __builtin_amdgcn_perm(a1, a0, 0x07030501u);
                const uint32_t th23 = __builtin_amdgcn_perm(a3, a2, 0x07030501u);
                const uint32_t tl01 = __builtin_amdgcn_perm(a1, a0, 0x06020400u);
                const uint32_t tl23 = __builtin_amdgcn_perm(a3, a2, 0x06020400u);
                const uint32_t d0 = 8 * c + 2 * q;
                // th01 = (a0.b1, a1.b1, a0.b3, a1.b3): the even element's high bytes of keys
                // 0, 1 in its low half, the odd element's in its high half
                *reinterpret_cast<uint32_t*>(vth + d0 * VS + p0) = __builtin_amdgcn_perm(th23, th01, 0x05040100u);
                *reinterpret_cast<uint32_t*>(vth + (d0 + 1) * VS + p0) = __builtin_amdgcn_perm(th23, th01, 0x07060302u);
                *reinterpret_cast<uint32_t*>(vtl + d0 * VS + p0) =
                    __builtin_amdgcn_perm(tl23, tl01, 0x05040100u) ^ 0x80808080u;
                *reinterpret_cast<uint32_t*>(vtl + (d0 + 1) * VS + p0) =
                    __builtin_amdgcn_perm(tl23, tl01, 0x07060302u) ^ 0x80808080u;
                vpart[2 * q] += (int)(int16_t)a0 + (int)(int16_t)a1 + (int)(int16_t)a2 + (int)(int16_t)a3;
                vpart[2 * q + 1] += ((int)a0 >> 16) + ((int)a1 >> 16) + ((int)a2 >> 16) + ((int)a3 >> 16);
            }
        }
#pragma unroll
        for (uint32_t q = 0; q < 8; q++) {
            int x = vpart[q];
            x += __shfl_xor(x, 4, 64);
            x += __shfl_xor(x, 8, 64);
            x += __shfl_xor(x, 16, 64);
            x += __shfl_xor(x, 32, 64);
            vpart[q] = x;
        }
        if (lane < 4) {
#pragma unroll
            for (uint32_t q = 0; q < 8; q++) vsw[w * 64 + HD * half + 8 * c + q] = vpart[q];
        }
    };

    // ---- K's byte limbs through LDS, 64 keys at a time in two buffers (the TAB's 16 KiB until
    // phase 2): a thread splits 16 d of one key (key 64 c + t / 4, d 16 (t % 4) ..), so the
    // workgroup reads K from global memory once instead of once per wavefront.  Buffer layout:
    // [2][hi, lo][64 keys][64 d] bytes.
    uint8_t* kbuf = lds;
    const uint32_t kk = t >> 2, kd = 16 * (t & 3);
    int4 kx0, kx1;
    auto load_kchunk = [&](uint32_t c) {
        const int16_t* kp = seq + (uint64_t)(64 * c + kk) * ld + k_off + kHd * h + kd;
        kx0 = *reinterpret_cast<const int4*>(kp);
        kx1 = *reinterpret_cast<const int4*>(kp + 8);
    };
    auto store_kchunk = [&](uint32_t c) {
        uint32_t h0, h1, h2, h3, l0, l1, l2, l3;
        limbs8(kx0, h0, h1, l0, l1);
        limbs8(kx1, h2, h3, l2, l3);
        uint8_t* bp = kbuf + (c & 1) * 8192 + kk * 64 + kd;
        *reinterpret_cast<uint4*>(bp) = make_uint4(h0, h1, h2, h3);
        *reinterpret_cast<uint4*>(bp + 4096) = make_uint4(l0, l1, l2, l3);
    };
    load_kchunk(0);
    stage_v(0);

    // ---- the wavefront's Q rows (B of phase 1): query qi, d 16 g .. 16 g + 15
    const uint32_t qi = q0 + 16 * w + c16;
    v4i qh, ql;
    limbs16(seq + (uint64_t)qi * ld + q_off + kHd * h + 16 * g, qh, ql);
    // The offset terms from MFMAs against ones (A' = A - 128 = 256 h + l):
    //   sum_d K Q = 2^16 HH + 2^8 MID + LL + 2^15 (sum h_K + sum h_Q) + 2^7 (sum l_K + sum l_Q) + 2^20,
    // the limb sums of Q (columns) once, those of K (rows) per key block on top of them.
    const v4i zero = {0, 0, 0, 0};
    const v4i ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
    const v4i c20 = {1 << 20, 1 << 20, 1 << 20, 1 << 20};
    const v4i qh1 = mfma(ones, qh, zero), ql1 = mfma(ones, ql, zero);

    // ---- phase 1: the scores, key block by key block, 4 blocks a chunk of K in LDS; chunk c
    // is written before the barrier that precedes its products, chunk c + 1 loaded under them
    int32_t sv[4 * KB];                 // register arrays: every index a constant (loops unrolled)
#pragma unroll
    for (uint32_t kb = 0; kb < KB; kb++) {
        if (kb % 4 == 0) {
            const uint32_t c = kb / 4;
            store_kchunk(c);
            __syncthreads();            // chunk c in LDS; every wavefront done with chunk c - 1
            if (c + 1 < KB / 4) load_kchunk(c + 1);
        }
        const uint8_t* kr = kbuf + ((kb / 4) & 1) * 8192 + (16 * (kb % 4) + c16) * 64 + 16 * g;
        const v4i kh = *reinterpret_cast<const v4i*>(kr);
        const v4i kl = *reinterpret_cast<const v4i*>(kr + 4096);
        const v4i hh = mfma(kh, qh, zero);
        v4i mid = mfma(kh, ql, zero);
        mid = mfma(kl, qh, mid);
        const v4i ll = mfma(kl, ql, c20);
        const v4i ha = mfma(kh, ones, qh1), la = mfma(kl, ones, ql1);
#pragma unroll
        for (uint32_t r = 0; r < 4; r++) {
            const uint32_t acc = ((uint32_t)hh[r] << 16) + ((uint32_t)mid[r] << 8) + (uint32_t)ll[r] +
                                 ((uint32_t)ha[r] << 15) + ((uint32_t)la[r] << 7);
            sv[4 * kb + r] = sat16_shr8((int32_t)acc);
            __asm__ volatile("" : "+v"(sv[4 * kb + r]));   // the score itself held, not its terms
        }
        // one key block at a time: left free, the scheduler gathers the blocks' MFMAs and spills
        __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();                                   // every wavefront done with the K chunks
    // the TAB straight into LDS (global_load_lds: no registers, four 16-byte copies a lane in
    // flight at once), then this wave's copies waited for
#pragma unroll
    for (uint32_t q = 0; q < 4; q++)
        __builtin_amdgcn_global_load_lds(tab + 4 * (t + 256 * q),
                                         (__attribute__((address_space(3))) void*)(stab + 4 * (64 * w + 256 * q)), 16, 0, 0);
    __builtin_amdgcn_s_waitcnt(0x0070);
    __syncthreads();                                   // TAB, V^T planes and V sums staged

    // ---- phase 2: the softmax over the T keys of the lane's query (its lane group g = 0..3)
    int32_t mx = -32768;
#pragma unroll
    for (uint32_t n = 0; n < 4 * KB; n++) mx = max(mx, sv[n]);
    mx = max(mx, __shfl_xor(mx, 16, 64));
    mx = max(mx, __shfl_xor(mx, 32, 64));
    // e(d), d = max - s: below dlim y = (d Cm) >> Cs < 2^17 and e = TAB[y & 4095] >> (y >> 12);
    // from dlim on e = 0 (TAB <= 2^16)
    const uint32_t cs = cfg & 63u, fp = (cfg >> 8) & 31u;
    const uint64_t cm24 = cm & 0xFFFFFFu;
    uint32_t part = 0;
#pragma unroll
    for (uint32_t n = 0; n < 4 * KB; n++) {
        const uint32_t d = (uint32_t)(mx - sv[n]);
        const uint32_t y = (uint32_t)(((uint64_t)d * cm24) >> cs);
        const uint32_t e = ((uint32_t)stab[y & 4095] >> ((y >> 12) & 31)) & (d < dlim ? ~0u : 0u);   // no branch
        sv[n] = (int32_t)e;
        part += e;
    }
    part += __shfl_xor(part, 16, 64);
    part += __shfl_xor(part, 32, 64);
    // P = min(floor(e R 2^(fp - 40) + 1/2), 32767), R = floor(2^40 / S): e <= S, so e R <= 2^40
    // and e R 2^(fp - 40) + 1/2 has at most 41 significant bits, exact in double; the
    // conversion truncates (the floor of a positive value) and saturates
    const uint64_t R = ((uint64_t)1 << 40) / (uint64_t)(part ? part : 1u);
    const double rd = __builtin_ldexp((double)R, (int)fp - 40);
    int psum = 0;
#pragma unroll
    for (uint32_t n = 0; n < 4 * KB; n++) {
        sv[n] = (int32_t)__builtin_fmin(__builtin_fma((double)(uint32_t)sv[n], rd, 0.5), 32767.0);
        psum += sv[n];
    }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);                  // sum_j P[qi][j]

    // ---- phase 3: o^T[d][qi] over 4 blocks of 16 d, two per staged half of V^T
    // result lane: d = 16 mb + 4 g + r (o null: the planes alone)
    int16_t* orow = o != nullptr ? o + ((uint64_t)b * T + qi) * o_ld + kHd * h : nullptr;
    const uint64_t prow = (uint64_t)b * T + qi;
    int32_t osum = 0;                                                   // PL: the lane's 16 outputs' sum
#pragma unroll
    for (uint32_t half = 0; half < 2; half++) {
        if (half == 1) {
            __syncthreads();                           // every wavefront done with the first half
            stage_v(1);
            __syncthreads();
        }
        v4i ohh[2], omid[2], oll[2];
#pragma unroll
        for (uint32_t m = 0; m < 2; m++) ohh[m] = omid[m] = oll[m] = v4i{0, 0, 0, 0};
#pragma unroll
        for (uint32_t ks = 0; ks < KS; ks++) {
            // B: the lane's P of key blocks 4 ks + q, byte 4 q + r = key 16 (4 ks + q) + 4 g + r
            uint32_t ph[4], pl[4];
#pragma unroll
            for (uint32_t q = 0; q < 4; q++) {
                const uint32_t n = 4 * (4 * ks + q);
                const uint32_t p01 = (uint32_t)sv[n] | ((uint32_t)sv[n + 1] << 16);      // P in [0, 32767]
                const uint32_t p23 = (uint32_t)sv[n + 2] | ((uint32_t)sv[n + 3] << 16);
                ph[q] = __builtin_amdgcn_perm(p23, p01, 0x07050301u);
                pl[q] = __builtin_amdgcn_perm(p23, p01, 0x06040200u) ^ 0x80808080u;
            }
            const v4i bh4 = {(int)ph[0], (int)ph[1], (int)ph[2], (int)ph[3]};
            const v4i bl4 = {(int)pl[0], (int)pl[1], (int)pl[2], (int)pl[3]};
#pragma unroll
            for (uint32_t m = 0; m < 2; m++) {
                const uint32_t off = (16 * m + c16) * VS + 64 * ks + 16 * g;
                const v4i vh = *reinterpret_cast<const v4i*>(vth + off);
                const v4i vl = *reinterpret_cast<const v4i*>(vtl + off);
                ohh[m] = mfma(vh, bh4, ohh[m]);
                omid[m] = mfma(vh, bl4, omid[m]);
                omid[m] = mfma(vl, bh4, omid[m]);
                oll[m] = mfma(vl, bl4, oll[m]);
            }
        }
#pragma unroll
        for (uint32_t m = 0; m < 2; m++) {
            const uint32_t mb = 2 * half + m;
            uint32_t pk[2];
#pragma unroll
            for (uint32_t r = 0; r < 4; r += 2) {
                const uint32_t d = 16 * mb + 4 * g + r;
                const int32_t vs0 = vsw[d] + vsw[64 + d] + vsw[128 + d] + vsw[192 + d];
                const int32_t vs1 = vsw[d + 1] + vsw[65 + d] + vsw[129 + d] + vsw[193 + d];
                const uint32_t t0 = 128u * (uint32_t)(vs0 + psum) - 16384u * T;
                const uint32_t t1 = 128u * (uint32_t)(vs1 + psum) - 16384u * T;
                const int o0 = sat16_shr8(wrap_sum(ohh[m][r], omid[m][r], oll[m][r], t0));
                const int o1 = sat16_shr8(wrap_sum(ohh[m][r + 1], omid[m][r + 1], oll[m][r + 1], t1));
                pk[r / 2] = (uint32_t)(uint16_t)o0 | ((uint32_t)(uint16_t)o1 << 16);
            }
            if (orow != nullptr) *reinterpret_cast<uint2*>(orow + 16 * mb + 4 * g) = make_uint2(pk[0], pk[1]);
            if constexpr (PL) {
                const uint32_t col = kHd * h + 16 * mb + 4 * g;
                *reinterpret_cast<uint32_t*>(po.hi + prow * po.k + col) = __builtin_amdgcn_perm(pk[1], pk[0], 0x07050301u);
                *reinterpret_cast<uint32_t*>(po.lo + prow * po.k + col) =
                    __builtin_amdgcn_perm(pk[1], pk[0], 0x06040200u) ^ 0x80808080u;
                osum += (int32_t)(int16_t)(pk[0] & 0xFFFF) + ((int32_t)pk[0] >> 16) + (int32_t)(int16_t)(pk[1] & 0xFFFF) +
                        ((int32_t)pk[1] >> 16);
            }
        }
    }
    if constexpr (PL) {
        // the four lane groups g of query c16 hold its 64 outputs of this head
        osum += __shfl_xor(osum, 16, 64);
        osum += __shfl_xor(osum, 32, 64);
        if (g == 0) po.part[(uint64_t)h * po.lines + prow] = osum;
    }
}

template <uint32_t T, bool PL>
void* attention_fn() {
    return reinterpret_cast<void*>(&attention_kernel<T, PL>);
}

int run_attention(const int16_t* qkv, int16_t* o, uint32_t batch, uint32_t seq, uint32_t heads, uint32_t head_dim,
                  uint64_t ld, uint32_t q_off, uint32_t k_off, uint32_t v_off, uint64_t o_ld, uint32_t smx_cm,
                  uint32_t smx_cfg, void* planes, hipStream_t s) {
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    if (batch == 0 || heads == 0) return CM_OK;
    if (qkv == nullptr || (o == nullptr && planes == nullptr))
        return fail(CM_EINVAL, "attention: a null qkv, or a null o without planes");
    if (head_dim != kHd) return fail(CM_EINVAL, "attention: head_dim %u (the kernel takes 64)", head_dim);
    if (seq != 64 && seq != 128 && seq != 256 && seq != 384)
        return fail(CM_EINVAL, "attention: %u keys (64, 128, 256 or 384)", seq);
    if (!aligned16(qkv) || !aligned16(o) || (ld & 7) || (o_ld & 7) || (q_off & 7) || (k_off & 7) || (v_off & 7))
        return fail(CM_EALIGN, "attention: rows and head columns must be 16-byte aligned");
    if (((smx_cfg >> 8) & 31u) > 39u || ((smx_cfg >> 8) & 31u) == 0u)
        return fail(CM_EINVAL, "attention: softmax output bits %u", (smx_cfg >> 8) & 31u);
    if ((uint64_t)batch * heads > 65535) return fail(CM_EINVAL, "attention: %u sequence-head pairs", batch * heads);
    if (planes != nullptr && (o_ld != (uint64_t)heads * kHd || heads > 64 || (reinterpret_cast<uintptr_t>(planes) & 255)))
        return fail(CM_EINVAL, "attention planes: o rows of exactly heads x 64 (at most 64 heads), 256-byte aligned "
                               "planes");
    const size_t lds = 16384 + 2 * (size_t)(kHd / 2) * (seq + 16) + 4 * 64 * sizeof(int32_t);
    if (lds > st->lds_per_block) return fail(CM_EINVAL, "attention: %zu bytes of LDS per workgroup", lds);
    const uint32_t dlim = smx_dlim(smx_cm & 0xFFFFFFu, smx_cfg & 63u);
    const dim3 grid(seq / kQb, batch * heads);
    const APlanes po = planes != nullptr ? a_planes_view(planes, batch * seq, heads * kHd, heads) : APlanes{};
#define CM_ATT(T, PL)                                                                                           \
    {                                                                                                           \
        static bool attr = false;                                                                               \
        if (!attr) {                                                                                            \
            CM_HIP_CHECK(hipFuncSetAttribute(attention_fn<T, PL>(), hipFuncAttributeMaxDynamicSharedMemorySize, \
                                             (int)lds));                                                        \
            attr = true;                                                                                        \
        }                                                                                                       \
        CM_LAUNCH("attention_kernel", (attention_kernel<T, PL>), grid, dim3(256), lds, s, qkv, o, st->smx_tab,  \
                  heads, ld, q_off, k_off, v_off, o_ld, smx_cm, smx_cfg, dlim, po);                             \
        return CM_OK;                                                                                           \
    }
#define CM_ATT_T(T) \
    case T: if (planes != nullptr) CM_ATT(T, true) else CM_ATT(T, false)
    switch (seq) {
        CM_ATT_T(64) CM_ATT_T(128) CM_ATT_T(256) CM_ATT_T(384)
    default: break;
    }
#undef CM_ATT_T
#undef CM_ATT
    return fail(CM_EINVAL, "attention: %u keys", seq);
}

}  // namespace
}  // namespace cm

extern "C" int cm_attention(const int16_t* qkv, int16_t* o, uint32_t batch, uint32_t seq, uint32_t heads,
                            uint32_t head_dim, uint64_t ld, uint32_t q_off, uint32_t k_off, uint32_t v_off,
                            uint64_t o_ld, uint32_t smx_cm, uint32_t smx_cfg, void* stream) {
    return cm::run_attention(qkv, o, batch, seq, heads, head_dim, ld, q_off, k_off, v_off, o_ld, smx_cm, smx_cfg,
                             nullptr, cm::as_stream(stream));
}

extern "C" int cm_attention_planes(const int16_t* qkv, int16_t* o, uint32_t batch, uint32_t seq, uint32_t heads,
                                   uint32_t head_dim, uint64_t ld, uint32_t q_off, uint32_t k_off, uint32_t v_off,
                                   uint32_t smx_cm, uint32_t smx_cfg, void* planes, void* stream) {
    if (planes == nullptr) return cm::fail(CM_EINVAL, "attention planes: no planes buffer");
    return cm::run_attention(qkv, o, batch, seq, heads, head_dim, ld, q_off, k_off, v_off, (uint64_t)heads * 64,
                             smx_cm, smx_cfg, planes, cm::as_stream(stream));
}
