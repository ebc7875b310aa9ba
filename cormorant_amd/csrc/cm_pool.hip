// cm_pool.hip -- the Pooling unit: MAX / AVG / LP1 / LP2 over NCHW planes.
//
// Windowed pools: one thread per output element, neighbouring threads on neighbouring
// output columns so that a tap's loads across a wavefront are one contiguous run of the
// input row (stride stride_w).  Global pools (a window as large as the plane, the
// MobileNet GlobalAveragePool 7x7 case) use one wavefront per output: the plane is read
// 64 lanes at a time and reduced across the wavefront.
#include "cm_common.h"

#include <algorithm>

namespace cm {
namespace {

__device__ __forceinline__ int sat16l(long long v) {
    return v > 32767 ? 32767 : (v < -32768 ? -32768 : (int)v);
}

// _pool_poly_sqrt (_simulate.py:230-272) on the exact sum S of squares (value S * 2^-16):
// S = m 4^k 2^16, m in [1, 4) cut to 16 fraction bits; Horner with the 2^-15 coefficients
// 252, -3091, 21076, 14529, every partial floored at 2^-20; the result 2^k * t floored at
// 2^-16.  Returns the result at 2^-16.
__device__ __forceinline__ long long poly_sqrt(long long S) {
    if (S <= 0) return 0;
    const int e = 63 - __clzll((unsigned long long)S);
    const int d = e - 16;
    const int k = d >= 0 ? d / 2 : -((-d + 1) / 2);
    const long long M = 2 * k >= 0 ? (S >> (2 * k)) : (S << (-2 * k));
    const long long T1 = (252LL * M - 3091LL * 65536) >> 11;
    const long long T2 = (T1 * M + 21076LL * 2097152) >> 16;
    const long long T3 = (T2 * M + 14529LL * 2097152) >> 16;
    return k >= 4 ? (T3 << (k - 4)) : (T3 >> (4 - k));
}

struct PoolGeom {
    uint32_t in_h, in_w, out_h, out_w, ph, pw, sh, sw, pt, pl, dh, dw, type, lp, cip;
};

// The pooled value of one window from its running max / sum and the count of valid taps
// (_simulate.py:275-358 then truncate).
__device__ __forceinline__ int finish(const PoolGeom& g, long long mx, long long sum, uint32_t valid) {
    if (g.type == 0) return valid ? (int)mx : -32768;
    if (g.type == 1) {
        long long d = g.cip ? (long long)g.ph * g.pw : (long long)valid;
        if (d < 1) d = 1;
        const long long inv = ((1LL << 23) + d / 2) / d;
        return sat16l((sum * inv) >> 23);
    }
    if (g.lp == 1) return sat16l(sum);
    return sat16l(poly_sqrt(sum) >> 8);
}

__device__ __forceinline__ void tap(const PoolGeom& g, long long v, long long& mx, long long& sum) {
    mx = v > mx ? v : mx;
    if (g.type == 1) sum += v;
    else if (g.type == 2) sum += g.lp == 1 ? (v < 0 ? -v : v) : v * v;
}

__device__ __forceinline__ uint32_t pack_i16(int lo, int hi) {
    return (uint32_t)(uint16_t)lo | ((uint32_t)(uint16_t)hi << 16);
}

__global__ __launch_bounds__(256) void pool_kernel(const int16_t* __restrict__ x,
                                                   int16_t* __restrict__ y, uint64_t total,
                                                   PoolGeom g) {
    for (uint64_t o = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; o < total;
         o += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t ow = (uint32_t)(o % g.out_w);
        const uint64_t t = o / g.out_w;
        const uint32_t oh = (uint32_t)(t % g.out_h);
        const uint64_t nc = t / g.out_h;
        const int16_t* xp = x + nc * g.in_h * g.in_w;
        long long mx = INT64_MIN, sum = 0;
        uint32_t valid = 0;
        for (uint32_t a = 0; a < g.ph; a++) {
            const long long ih = (long long)oh * g.sh + (long long)a * g.dh - g.pt;
            if (ih < 0 || ih >= g.in_h) continue;
            for (uint32_t b = 0; b < g.pw; b++) {
                const long long iw = (long long)ow * g.sw + (long long)b * g.dw - g.pl;
                if (iw < 0 || iw >= g.in_w) continue;
                valid++;
                tap(g, xp[ih * g.in_w + iw], mx, sum);
            }
        }
        y[o] = (int16_t)finish(g, mx, sum, valid);
    }
}

// Global pool (window == plane, stride 1, no padding, out 1x1): one wavefront per plane.
__global__ __launch_bounds__(256) void pool_global_kernel(const int16_t* __restrict__ x,
                                                          int16_t* __restrict__ y, uint64_t planes,
                                                          PoolGeom g) {
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t nc = (uint64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (nc >= planes) return;
    const uint32_t hw = g.in_h * g.in_w;
    const int16_t* xp = x + nc * hw;
    long long mx = INT64_MIN, sum = 0;
    for (uint32_t i = lane; i < hw; i += 64) tap(g, xp[i], mx, sum);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        long long om = __shfl_xor(mx, off, 64);
        mx = om > mx ? om : mx;
        sum += __shfl_xor(sum, off, 64);
    }
    if (lane == 0) y[nc] = (int16_t)finish(g, mx, sum, hw);
}

// Global pool over small planes (hw <= kSmallPlane): a lane owns a plane.  A workgroup's
// planes are contiguous, so it copies their elements into LDS with coalesced loads and
// each lane then reduces its own plane from LDS; the outputs leave as one contiguous run.
constexpr uint32_t kSmallPlane = 64;

__global__ __launch_bounds__(64) void pool_global_small_kernel(const int16_t* __restrict__ x,
                                                               int16_t* __restrict__ y, uint64_t planes,
                                                               PoolGeom g) {
    __shared__ __attribute__((aligned(16))) int16_t buf[64 * kSmallPlane];
    const uint32_t hw = g.in_h * g.in_w;
    const uint64_t p0 = (uint64_t)blockIdx.x * 64;
    const uint32_t np = (uint32_t)(planes - p0 < 64 ? planes - p0 : 64);
    const int16_t* xs = x + p0 * hw;
    if (np == 64 && aligned16(x)) {
        // 64 whole planes: 8 hw 16-byte words (128 hw bytes from a 16-byte aligned start), copied
        // straight into LDS (global_load_lds: every copy in flight at once, no registers)
        const uint32_t n4 = 8 * hw;
#pragma unroll
        for (uint32_t u = 0; u < kSmallPlane / 8; u++) {
            const uint32_t i = threadIdx.x + 64 * u;
            if (i < n4)
                __builtin_amdgcn_global_load_lds(xs + 8 * i, (__attribute__((address_space(3))) void*)(buf + 8 * 64 * u),
                                                 16, 0, 0);
        }
        __builtin_amdgcn_s_waitcnt(0x0070);
    } else {
        for (uint32_t i = threadIdx.x; i < np * hw; i += 64) buf[i] = xs[i];
    }
    __syncthreads();
    if (threadIdx.x >= np) return;
    const int16_t* xp = buf + threadIdx.x * hw;
    long long mx = INT64_MIN, sum = 0;
    for (uint32_t i = 0; i < hw; i++) tap(g, xp[i], mx, sum);
    y[p0 + threadIdx.x] = (int16_t)finish(g, mx, sum, hw);
}

// MAX / AVG 2x2 stride 2 without padding or dilation, on rows of 16k columns: a lane makes 8
// outputs of one row from two 16-byte words of each of its two input rows and writes them as
// one 16-byte word.  AVG divides by the window's 4 taps: (sum * round(2^23 / 4)) >> 23.
__global__ __launch_bounds__(256) void pool2x2_kernel(const int16_t* __restrict__ x, int16_t* __restrict__ y,
                                                      uint64_t items, uint32_t groups, PoolGeom g) {
    for (uint64_t it = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; it < items;
         it += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t row = it / groups;                       // plane * out_h + oh
        const uint32_t j = (uint32_t)(it - row * groups);
        const uint64_t plane = row / g.out_h;
        const uint32_t oh = (uint32_t)(row - plane * g.out_h);
        const int16_t* r0 = x + (plane * g.in_h + 2 * oh) * g.in_w + 16 * j;
        const int16_t* r1 = r0 + g.in_w;
        int4 v[4] = {*reinterpret_cast<const int4*>(r0), *reinterpret_cast<const int4*>(r0 + 8),
                     *reinterpret_cast<const int4*>(r1), *reinterpret_cast<const int4*>(r1 + 8)};
        const int16_t* a = reinterpret_cast<const int16_t*>(&v[0]);   // row 2 oh, 16 columns
        const int16_t* b = reinterpret_cast<const int16_t*>(&v[2]);   // row 2 oh + 1
        int q[8];
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const int x0 = a[2 * t], x1 = a[2 * t + 1], x2 = b[2 * t], x3 = b[2 * t + 1];
            if (g.type == 0) q[t] = max(max(x0, x1), max(x2, x3));
            else q[t] = (x0 + x1 + x2 + x3) >> 2;                    // (sum * 2^21) >> 23, in range
        }
        int4 o;
        o.x = (int)pack_i16(q[0], q[1]);
        o.y = (int)pack_i16(q[2], q[3]);
        o.z = (int)pack_i16(q[4], q[5]);
        o.w = (int)pack_i16(q[6], q[7]);
        store_stream(y + row * g.out_w + 8 * j, o);
    }
}

}  // namespace
}  // namespace cm

extern "C" int cm_pool(const int16_t* x, int16_t* y, uint32_t batch, uint32_t channels,
                       uint32_t in_h, uint32_t in_w, uint32_t out_h, uint32_t out_w,
                       uint32_t pool_h, uint32_t pool_w, uint32_t stride_h, uint32_t stride_w,
                       uint32_t pad_top, uint32_t pad_left, uint32_t dil_h, uint32_t dil_w,
                       uint32_t pool_type, uint32_t lp_order, uint32_t count_include_pad,
                       void* stream) {
    using namespace cm;
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    if (pool_type > 2) return fail(CM_EINVAL, "pool: pool_type %u", pool_type);
    if (pool_h == 0 || pool_w == 0 || stride_h == 0 || stride_w == 0 || dil_h == 0 || dil_w == 0)
        return fail(CM_EINVAL, "pool: zero window, stride or dilation");
    const uint64_t planes = (uint64_t)batch * channels;
    const uint64_t total = planes * out_h * out_w;
    if (total == 0) return CM_OK;
    PoolGeom g{in_h, in_w, out_h, out_w, pool_h, pool_w, stride_h, stride_w, pad_top, pad_left,
               dil_h, dil_w, pool_type, lp_order, count_include_pad};
    hipStream_t s = as_stream(stream);
    const bool global = out_h == 1 && out_w == 1 && pool_h == in_h && pool_w == in_w &&
                        pad_top == 0 && pad_left == 0 && dil_h == 1 && dil_w == 1;
    if (global && (uint64_t)in_h * in_w <= kSmallPlane) {
        CM_LAUNCH("pool_global_kernel", pool_global_small_kernel, dim3((unsigned)((planes + 63) / 64)), dim3(64), 0,
                  s, x, y, planes, g);
        return CM_OK;
    }
    if (pool_type <= 1 && pool_h == 2 && pool_w == 2 && stride_h == 2 && stride_w == 2 && dil_h == 1 &&
        dil_w == 1 && pad_top == 0 && pad_left == 0 && (in_w & 15) == 0 && out_w == in_w / 2 &&
        out_h <= in_h / 2 && aligned16(x) && aligned16(y)) {
        const uint32_t groups = out_w / 8;
        const uint64_t items = planes * out_h * groups;
        const unsigned blocks = (unsigned)std::min<uint64_t>((items + 255) / 256, 65536ull * 8);
        CM_LAUNCH("pool2x2_kernel", pool2x2_kernel, dim3(blocks), dim3(256), 0, s, x, y, items, groups, g);
        return CM_OK;
    }
    if (global) {
        CM_LAUNCH("pool_global_kernel", pool_global_kernel, dim3((unsigned)((planes + 3) / 4)), dim3(256), 0, s,
                           x, y, planes, g);
    } else {
        uint64_t blocks = (total + 255) / 256;
        if (blocks > 65536ull * 8) blocks = 65536ull * 8;
        CM_LAUNCH("pool_kernel", pool_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, y, total, g);
    }
    return CM_OK;
}
