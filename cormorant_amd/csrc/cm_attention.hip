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
// The int32 wrap makes every sum exact in any order, so v_dot2_i32_i16 (two products per
// lane-op, no clamp) forms them directly.  Workgroup: 4 wavefronts, lane = query, wavefront w
// = keys [w T/4, (w+1) T/4).
//   phase 1: the lane's Q row in registers, K rows read at wavefront-uniform addresses;
//   phase 2: the softmax: row max and sum across the four wavefronts through LDS,
//            e = TAB[y & 4095] >> (y >> 12), y = (max - s) Cm >> Cs, R = floor(2^40 / S),
//            P = min((e R + 2^(39 - fp)) >> (40 - fp), 32767) (the unit's integer rule);
//   phase 3: o partials over the wavefront's keys from V transposed in LDS (k pairs of one
//            d contiguous: 16-byte broadcast reads of 4 key pairs), summed across the
//            wavefronts through LDS (the region V used), then the output rule.
// LDS: TAB (16 KiB) + one 64 KiB region (V^T [64][T] and the max / sum exchange, then the
// partials [4][64][64]): two workgroups per compute unit.  T <= 384.
#include "cm_common.h"

#include <algorithm>

namespace cm {
namespace {

constexpr uint32_t kHd = 64;                 // head dimension
constexpr uint32_t kQb = 64;                 // queries per workgroup
constexpr uint32_t kRegion = 65536;          // bytes: V^T (T <= 384) + exchange, or the partials

typedef short v2s __attribute__((ext_vector_type(2)));

__device__ __forceinline__ int dot2(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(v2s, a), __builtin_bit_cast(v2s, b), c, false);
}

__device__ __forceinline__ int sat16_shr8(int acc) { return min(max(acc >> 8, -32768), 32767); }

// NK = keys per wavefront (T / 4).  qkv rows: ld elements apart; Q / K / V of head h at
// columns q_off / k_off / v_off + 64 h.  o rows: o_ld apart, head h at columns 64 h.
template <uint32_t NK>
__global__ __launch_bounds__(256, 2) void attention_kernel(const int16_t* __restrict__ qkv, int16_t* __restrict__ o,
                                                           const int32_t* __restrict__ tab, uint32_t heads,
                                                           uint64_t ld, uint32_t q_off, uint32_t k_off,
                                                           uint32_t v_off, uint64_t o_ld, uint32_t cm, uint32_t cfg) {
    constexpr uint32_t T = 4 * NK;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    int32_t* stab = reinterpret_cast<int32_t*>(lds);                     // [4096]
    uint8_t* region = lds + 16384;
    int16_t* vt = reinterpret_cast<int16_t*>(region);                     // [64][T]
    uint32_t* xch = reinterpret_cast<uint32_t*>(region + 2 * kHd * T);    // [2][4][64], past V^T
    int32_t* red = reinterpret_cast<int32_t*>(region);                    // [4][64][64]

    const uint32_t t = threadIdx.x, lane = t & 63, w = t >> 6;
    const uint32_t bh = blockIdx.y, b = bh / heads, h = bh - b * heads;
    const uint32_t q0 = blockIdx.x * kQb;
    const int16_t* seq = qkv + (uint64_t)b * T * ld;

    // ---- staging: TAB, V^T, the lane's Q row
    for (uint32_t e = t; e < 1024; e += 256)
        reinterpret_cast<int4*>(stab)[e] = reinterpret_cast<const int4*>(tab)[e];
    for (uint32_t e = t; e < T * (kHd / 8); e += 256) {
        const uint32_t j = e >> 3, d0 = (e & 7) * 8;
        const int4 v = *reinterpret_cast<const int4*>(seq + (uint64_t)j * ld + v_off + kHd * h + d0);
        const int16_t* vv = reinterpret_cast<const int16_t*>(&v);
#pragma unroll
        for (uint32_t q = 0; q < 8; q++) vt[(d0 + q) * T + j] = vv[q];
    }
    const uint32_t qi = q0 + lane;
    const bool qlive = qi < T;
    uint32_t qr[kHd / 2];
    {
        const int16_t* qrow = seq + (uint64_t)(qlive ? qi : 0) * ld + q_off + kHd * h;
#pragma unroll
        for (uint32_t c = 0; c < kHd / 8; c++) {
            const int4 v = *reinterpret_cast<const int4*>(qrow + 8 * c);
            qr[4 * c] = v.x; qr[4 * c + 1] = v.y; qr[4 * c + 2] = v.z; qr[4 * c + 3] = v.w;
        }
    }

    // ---- phase 1: scores of the wavefront's keys (K rows at wavefront-uniform addresses:
    // scalar loads)
    const uint32_t j0 = __builtin_amdgcn_readfirstlane(w * NK);
    int32_t sv[NK];                    // register arrays: every index a constant (loops unrolled)
#pragma unroll
    for (uint32_t n = 0; n < NK; n++) {
        const int16_t* krow = seq + (uint64_t)(j0 + n) * ld + k_off + kHd * h;
        int acc = 0;
#pragma unroll
        for (uint32_t c = 0; c < kHd / 8; c++) {
            const int4 kv = *reinterpret_cast<const int4*>(krow + 8 * c);
            acc = dot2(qr[4 * c], kv.x, acc);
            acc = dot2(qr[4 * c + 1], kv.y, acc);
            acc = dot2(qr[4 * c + 2], kv.z, acc);
            acc = dot2(qr[4 * c + 3], kv.w, acc);
        }
        sv[n] = sat16_shr8(acc);
    }

    // ---- phase 2: the softmax over all T keys of the lane's query
    int32_t mx = -32768;
#pragma unroll
    for (uint32_t n = 0; n < NK; n++) mx = max(mx, sv[n]);
    xch[w * 64 + lane] = (uint32_t)mx;
    __syncthreads();                                                     // also: TAB and V^T staged
    mx = max(max((int32_t)xch[lane], (int32_t)xch[64 + lane]), max((int32_t)xch[128 + lane], (int32_t)xch[192 + lane]));
    const uint32_t cs = cfg & 63u, fp = (cfg >> 8) & 31u;
    const uint64_t cm24 = cm & 0xFFFFFFu;
    uint32_t part = 0;
#pragma unroll
    for (uint32_t n = 0; n < NK; n++) {
        const uint64_t y = ((uint64_t)(uint32_t)(mx - sv[n]) * cm24) >> cs;
        const uint64_t sh = y >> 12;
        const uint32_t e = sh >= 63 ? 0u : (uint32_t)((uint64_t)(uint32_t)stab[y & 4095] >> sh);
        sv[n] = (int32_t)e;
        part += e;
    }
    xch[256 + w * 64 + lane] = part;
    __syncthreads();
    const uint32_t S = xch[256 + lane] + xch[320 + lane] + xch[384 + lane] + xch[448 + lane];
    const uint64_t R = ((uint64_t)1 << 40) / (uint64_t)(S ? S : 1u);
    const uint32_t psh = 40 - fp;
    const uint64_t half = (uint64_t)1 << (psh - 1);
    uint32_t pp[NK / 2];                                                 // (P[j], P[j+1]) pairs
#pragma unroll
    for (uint32_t n = 0; n < NK; n += 2) {
        const uint64_t a = ((uint64_t)(uint32_t)sv[n] * R + half) >> psh;
        const uint64_t c = ((uint64_t)(uint32_t)sv[n + 1] * R + half) >> psh;
        const uint32_t pa = a > 32767 ? 32767u : (uint32_t)a, pc = c > 32767 ? 32767u : (uint32_t)c;
        pp[n / 2] = pa | (pc << 16);
    }

    // ---- phase 3: o over the wavefront's keys from V^T (k pairs of one d contiguous)
    int32_t acc[kHd];
#pragma unroll
    for (uint32_t d = 0; d < kHd; d++) acc[d] = 0;
#pragma unroll
    for (uint32_t g = 0; g < NK / 8; g++) {
        const uint32_t p0 = pp[4 * g], p1 = pp[4 * g + 1], p2 = pp[4 * g + 2], p3 = pp[4 * g + 3];
        const int16_t* vcol = vt + j0 + 8 * g;
#pragma unroll
        for (uint32_t d = 0; d < kHd; d++) {
            const uint4 v = *reinterpret_cast<const uint4*>(vcol + d * T);
            acc[d] = dot2(p3, v.w, dot2(p2, v.z, dot2(p1, v.y, dot2(p0, v.x, acc[d]))));
        }
    }
    __syncthreads();                                                     // V^T done: the region is the partials
#pragma unroll
    for (uint32_t d = 0; d < kHd; d += 4)
        *reinterpret_cast<int4*>(red + (w * 64 + lane) * kHd + d) = make_int4(acc[d], acc[d + 1], acc[d + 2], acc[d + 3]);
    __syncthreads();
    // thread t: query t / 4, 16 d from 16 (t % 4)
    const uint32_t i = t >> 2, d0 = (t & 3) * 16;
    if (q0 + i < T) {
        uint32_t out[8];
#pragma unroll
        for (uint32_t d = 0; d < 16; d += 2) {
            uint32_t s0 = 0, s1 = 0;
#pragma unroll
            for (uint32_t ww = 0; ww < 4; ww++) {
                s0 += (uint32_t)red[(ww * 64 + i) * kHd + d0 + d];
                s1 += (uint32_t)red[(ww * 64 + i) * kHd + d0 + d + 1];
            }
            out[d / 2] = (uint32_t)(uint16_t)sat16_shr8((int)s0) | ((uint32_t)(uint16_t)sat16_shr8((int)s1) << 16);
        }
        int16_t* orow = o + ((uint64_t)b * T + q0 + i) * o_ld + kHd * h + d0;
        *reinterpret_cast<uint4*>(orow) = make_uint4(out[0], out[1], out[2], out[3]);
        *reinterpret_cast<uint4*>(orow + 8) = make_uint4(out[4], out[5], out[6], out[7]);
    }
}

template <uint32_t NK>
void* attention_fn() {
    return reinterpret_cast<void*>(&attention_kernel<NK>);
}

}  // namespace
}  // namespace cm

extern "C" int cm_attention(const int16_t* qkv, int16_t* o, uint32_t batch, uint32_t seq, uint32_t heads,
                            uint32_t head_dim, uint64_t ld, uint32_t q_off, uint32_t k_off, uint32_t v_off,
                            uint64_t o_ld, uint32_t smx_cm, uint32_t smx_cfg, void* stream) {
    using namespace cm;
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    if (batch == 0 || heads == 0) return CM_OK;
    if (head_dim != kHd) return fail(CM_EINVAL, "attention: head_dim %u (the kernel takes 64)", head_dim);
    if (seq != 64 && seq != 128 && seq != 256 && seq != 384)
        return fail(CM_EINVAL, "attention: %u keys (64, 128, 256 or 384)", seq);
    if (!aligned16(qkv) || !aligned16(o) || (ld & 7) || (o_ld & 7) || (q_off & 7) || (k_off & 7) || (v_off & 7))
        return fail(CM_EALIGN, "attention: rows and head columns must be 16-byte aligned");
    if (((smx_cfg >> 8) & 31u) > 39u || ((smx_cfg >> 8) & 31u) == 0u)
        return fail(CM_EINVAL, "attention: softmax output bits %u", (smx_cfg >> 8) & 31u);
    if ((uint64_t)batch * heads > 65535) return fail(CM_EINVAL, "attention: %u sequence-head pairs", batch * heads);
    const size_t lds = 16384 + kRegion;
    if (lds > st->lds_per_block) return fail(CM_EINVAL, "attention: %zu bytes of LDS per workgroup", lds);
    hipStream_t s = as_stream(stream);
    const dim3 grid((seq + kQb - 1) / kQb, batch * heads);
#define CM_ATT(NK)                                                                                              \
    case 4 * NK: {                                                                                              \
        static bool attr = false;                                                                               \
        if (!attr) {                                                                                            \
            CM_HIP_CHECK(hipFuncSetAttribute(attention_fn<NK>(), hipFuncAttributeMaxDynamicSharedMemorySize,    \
                                             (int)lds));                                                        \
            attr = true;                                                                                        \
        }                                                                                                       \
        CM_LAUNCH("attention_kernel", attention_kernel<NK>, grid, dim3(256), lds, s, qkv, o, st->smx_tab,      \
                  heads, ld, q_off, k_off, v_off, o_ld, smx_cm, smx_cfg);                                       \
        return CM_OK;                                                                                           \
    }
    switch (seq) {
        CM_ATT(16) CM_ATT(32) CM_ATT(64) CM_ATT(96)
    default: break;
    }
#undef CM_ATT
    return fail(CM_EINVAL, "attention: %u keys", seq);
}
