// cm_layout.hip -- data movement between the units' layouts: a 4-D strided int16 gather,
// dst contiguous [d0][d1][d2][d3] from src element i0 s0 + i1 s1 + i2 s2 + i3 s3.  The
// attention uses it to split the projections into per-head operands (the q image
// transposed per head, the K / V rows of a head) and to merge the heads' outputs back into
// token rows: the moves the reference's VitAttnPrep / LlmAttnMerge make between the
// projection MatMuls and the attention contractions.
//
// cm_copy16 is the same gather into a strided destination (the KV-cache row writes).
//
// Three kernels by the strides:
//   * the innermost dimension contiguous in src (s3 == 1), rows of whole 16-byte words: one
//     lane per 16-byte word, loads and stores both whole words;
//   * dimensions 2 and 3 transposed (s2 == 1): 64 x 64 tiles through LDS, read 128 bytes per
//     src row and written 128 bytes per dst row;
//   * anything else: one lane per element.
#include "cm_common.h"

#include <algorithm>

namespace cm {
namespace {

struct Perm {
    uint32_t d0, d1, d2, d3;
    uint64_t s0, s1, s2, s3;
};

__global__ __launch_bounds__(256) void permute_words_kernel(const int16_t* __restrict__ src, int16_t* __restrict__ dst,
                                                            uint64_t words, Perm p) {
    const uint32_t w3 = p.d3 >> 3;
    for (uint64_t w = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; w < words;
         w += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t r = w / w3;                      // dst row (i0, i1, i2)
        const uint32_t j = (uint32_t)(w - r * w3);
        const uint64_t r01 = r / p.d2;
        const uint32_t i2 = (uint32_t)(r - r01 * p.d2);
        const uint64_t i0 = r01 / p.d1;
        const uint32_t i1 = (uint32_t)(r01 - i0 * p.d1);
        const int4 v = *reinterpret_cast<const int4*>(src + i0 * p.s0 + i1 * p.s1 + i2 * p.s2 + 8ull * j);
        store_stream(dst + 8 * w, v);
    }
}

// dst[i0][i1][i2][i3] = src[i0 s0 + i1 s1 + i2 + i3 s3]: tile (i2 0..63, i3 0..63) of one
// (i0, i1) plane; blockIdx.x = tile of the plane, blockIdx.y = plane.
__global__ __launch_bounds__(256) void permute_tile_kernel(const int16_t* __restrict__ src, int16_t* __restrict__ dst,
                                                           uint32_t tiles2, Perm p) {
    __shared__ int16_t tile[64][66];
    const uint32_t plane = blockIdx.y, i1 = plane % p.d1, i0 = plane / p.d1;
    const uint32_t t2 = blockIdx.x % tiles2, t3 = blockIdx.x / tiles2;
    const uint32_t a2 = 64 * t2, a3 = 64 * t3;
    const int16_t* sp = src + i0 * p.s0 + i1 * p.s1;
    const uint32_t lane = threadIdx.x & 63, grp = threadIdx.x >> 6;
    // read: src rows i3 (64 of them), 64 consecutive i2 each
#pragma unroll 4
    for (uint32_t r = grp; r < 64; r += 4) {
        const uint32_t i3 = a3 + r, i2 = a2 + lane;
        tile[r][lane] = (i3 < p.d3 && i2 < p.d2) ? sp[(uint64_t)i3 * p.s3 + i2] : (int16_t)0;
    }
    __syncthreads();
    int16_t* dp = dst + ((uint64_t)plane * p.d2) * p.d3;
#pragma unroll 4
    for (uint32_t r = grp; r < 64; r += 4) {
        const uint32_t i2 = a2 + r, i3 = a3 + lane;
        if (i2 < p.d2 && i3 < p.d3) dp[(uint64_t)i2 * p.d3 + i3] = tile[lane][r];
    }
}

__global__ __launch_bounds__(256) void permute_elems_kernel(const int16_t* __restrict__ src, int16_t* __restrict__ dst,
                                                            uint64_t total, Perm p) {
    for (uint64_t e = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (uint64_t)gridDim.x * blockDim.x) {
        uint64_t r = e;
        const uint32_t i3 = (uint32_t)(r % p.d3);
        r /= p.d3;
        const uint32_t i2 = (uint32_t)(r % p.d2);
        r /= p.d2;
        const uint32_t i1 = (uint32_t)(r % p.d1);
        const uint64_t i0 = r / p.d1;
        dst[e] = src[i0 * p.s0 + i1 * p.s1 + i2 * p.s2 + i3 * p.s3];
    }
}

// dst[i0 t0 + i1 t1 + i2 t2 + i3 t3] = src[i0 s0 + i1 s1 + i2 s2 + i3 s3]: a lane per element.
__global__ __launch_bounds__(256) void copy_elems_kernel(const int16_t* __restrict__ src, int16_t* __restrict__ dst,
                                                         uint64_t total, Perm p, Perm q) {
    for (uint64_t e = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (uint64_t)gridDim.x * blockDim.x) {
        uint64_t r = e;
        const uint32_t i3 = (uint32_t)(r % p.d3);
        r /= p.d3;
        const uint32_t i2 = (uint32_t)(r % p.d2);
        r /= p.d2;
        const uint32_t i1 = (uint32_t)(r % p.d1);
        const uint64_t i0 = r / p.d1;
        dst[i0 * q.s0 + i1 * q.s1 + i2 * q.s2 + i3 * q.s3] = src[i0 * p.s0 + i1 * p.s1 + i2 * p.s2 + i3 * p.s3];
    }
}

unsigned grid_of(uint64_t items) {
    return (unsigned)std::max<uint64_t>(1, std::min<uint64_t>((items + 255) / 256, 65536ull * 8));
}

}  // namespace
}  // namespace cm

extern "C" int cm_permute16(const int16_t* src, int16_t* dst, uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3,
                            uint64_t s0, uint64_t s1, uint64_t s2, uint64_t s3, void* stream) {
    using namespace cm;
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    const uint64_t total = (uint64_t)d0 * d1 * d2 * d3;
    if (total == 0) return CM_OK;
    hipStream_t s = as_stream(stream);
    const Perm p{d0, d1, d2, d3, s0, s1, s2, s3};
    if (s3 == 1 && (d3 & 7) == 0 && aligned16(src) && aligned16(dst) && (s0 & 7) == 0 && (s1 & 7) == 0 &&
        (s2 & 7) == 0) {
        CM_LAUNCH("permute_words_kernel", permute_words_kernel, dim3(grid_of(total / 8)), dim3(256), 0, s, src, dst,
                  total / 8, p);
        return CM_OK;
    }
    if (s2 == 1 && (uint64_t)d0 * d1 < 65536) {
        const uint32_t tiles2 = (d2 + 63) / 64, tiles3 = (d3 + 63) / 64;
        if ((uint64_t)tiles2 * tiles3 < 0x7FFFFFFFull) {
            CM_LAUNCH("permute_tile_kernel", permute_tile_kernel, dim3(tiles2 * tiles3, d0 * d1), dim3(256), 0, s, src,
                      dst, tiles2, p);
            return CM_OK;
        }
    }
    CM_LAUNCH("permute_elems_kernel", permute_elems_kernel, dim3(grid_of(total)), dim3(256), 0, s, src, dst, total, p);
    return CM_OK;
}

extern "C" int cm_copy16(const int16_t* src, int16_t* dst, uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3,
                         uint64_t s0, uint64_t s1, uint64_t s2, uint64_t s3, uint64_t t0, uint64_t t1, uint64_t t2,
                         uint64_t t3, void* stream) {
    using namespace cm;
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    const uint64_t total = (uint64_t)d0 * d1 * d2 * d3;
    if (total == 0) return CM_OK;
    const Perm p{d0, d1, d2, d3, s0, s1, s2, s3}, q{d0, d1, d2, d3, t0, t1, t2, t3};
    CM_LAUNCH("copy_elems_kernel", copy_elems_kernel, dim3(grid_of(total)), dim3(256), 0, as_stream(stream), src, dst,
              total, p, q);
    return CM_OK;
}

// ---------------------------------------------------------------- embedding rows
// out[t][0 .. d) = table[clamp(ids[t], 0, rows - 1)][0 .. d) as 32-bit lanes: a workgroup per id,
// four lanes a thread per step (one 16-byte store); int16 table lanes are sign-extended.
namespace cm {
namespace {

template <bool I16>
__global__ __launch_bounds__(256) void embed_rows_kernel(const void* __restrict__ table, const int32_t* __restrict__ ids,
                                                         int32_t* __restrict__ out, uint32_t rows, uint32_t d) {
    const uint32_t t = blockIdx.x;
    int32_t id = ids[t];
    id = id < 0 ? 0 : (id >= (int32_t)rows ? (int32_t)rows - 1 : id);
    int32_t* o = out + (uint64_t)t * d;
    for (uint32_t c = 4 * threadIdx.x; c < d; c += 4 * blockDim.x) {
        int4 v;
        if (I16) {
            const short4 s = *reinterpret_cast<const short4*>(static_cast<const int16_t*>(table) + (uint64_t)id * d + c);
            v = make_int4(s.x, s.y, s.z, s.w);
        } else {
            v = *reinterpret_cast<const int4*>(static_cast<const int32_t*>(table) + (uint64_t)id * d + c);
        }
        *reinterpret_cast<int4*>(o + c) = v;
    }
}

}  // namespace
}  // namespace cm

extern "C" int cm_embed_rows(const void* table, uint32_t table_i16, const int32_t* ids, void* out, uint32_t n_ids,
                             uint32_t rows, uint32_t d, void* stream) {
    using namespace cm;
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    if (n_ids == 0 || d == 0) return CM_OK;
    if (rows == 0) return fail(CM_EINVAL, "embed: an empty table");
    if (n_ids > 0x7FFFFFFFu) return fail(CM_EINVAL, "embed: %u ids", n_ids);
    if ((d & 3) || !aligned16(out) || (reinterpret_cast<uintptr_t>(table) & (table_i16 ? 7 : 15)) ||
        (reinterpret_cast<uintptr_t>(ids) & 3))
        return fail(CM_EALIGN, "embed: rows of a multiple of 4 lanes, 16-byte aligned out and table rows");
    hipStream_t s = as_stream(stream);
    if (table_i16) {
        CM_LAUNCH("embed_rows_kernel", embed_rows_kernel<true>, dim3(n_ids), dim3(256), 0, s, table, ids,
                  static_cast<int32_t*>(out), rows, d);
    } else {
        CM_LAUNCH("embed_rows_kernel", embed_rows_kernel<false>, dim3(n_ids), dim3(256), 0, s, table, ids,
                  static_cast<int32_t*>(out), rows, d);
    }
    return CM_OK;
}
