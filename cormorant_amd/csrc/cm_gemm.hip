// cm_gemm.hip -- exact int16 x int16 contractions on CDNA4 i8 MFMA: the Matmul unit and
// the standard (group 1) Conv unit as an implicit GEMM; the depthwise conv runs direct.
//
// Arithmetic.  Every int16 operand x is written x - 128 = 256 h + l with h = x >> 8 and
// l = (x & 255) - 128, both signed bytes (the low byte with its top bit flipped).  Then
//   sum_k a b = sum_k A'B' + 128 sum_k a + 128 sum_k b - 16384 K,   A' = a - 128, B' = b - 128
//   sum_k A'B' = 2^16 HH + 2^8 (HL + LH) + LL
// where HH, HL, LH, LL are sums of byte products, each exact in int32 (|h l| <= 2^14, so
// K <= 32768 keeps HL + LH below 2^31).  Per 32 x 32 block and 32-k substep, four
// v_mfma_i32_32x32x32_i8 accumulate HH, MID = HL + LH and LL; the epilogue recombines them
// with the row / column sums in int32 (int64 only for K > 8192 on the saturating path) and
// applies the unit's output rule: floor(acc / 2^8) saturated to int16, after an int32 wrap
// for the power-of-two path.  Padding of k (beyond K or past the channels of a conv tile)
// is the byte pair (0, 0) -- A' = 0 -- on both sides and is left out of the sums, so it
// contributes nothing.
//
// Data flow: split kernels write the two byte planes of A as [rows][kp] and of B as
// [cols][kp] (k contiguous, the MFMA operand order; B transposed in registers or LDS), plus
// per-1024-k partial row / column sums; the plane GEMM streams 64-k tiles of the four planes
// into LDS with direct global -> LDS copies and sums the partials in its prologue.
#include "cm_common.h"
#include "cm_rowops_math.h"

namespace cm {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int BN = 128, BK = 64;               // output tile columns; k step in elements (= plane bytes)
constexpr int SLAB = 1024;                     // k per partial-sum slab

// Where batch slice bt of an operand starts: (bt / inner) s1 + (bt % inner) s2 elements (the
// (sequence, head) pairs of an attention's operands inside one projection), or bt s1.
struct Slices {
    uint64_t s1 = 0, s2 = 0;
    uint32_t inner = 1;
    __host__ __device__ uint64_t off(uint32_t bt) const {
        return inner > 1 ? (uint64_t)(bt / inner) * s1 + (uint64_t)(bt % inner) * s2 : (uint64_t)bt * s1;
    }
};

__device__ __forceinline__ uint32_t pack_hi(const int16_t* v) {   // 4 high bytes
    return (uint32_t)(uint8_t)(v[0] >> 8) | ((uint32_t)(uint8_t)(v[1] >> 8) << 8) |
           ((uint32_t)(uint8_t)(v[2] >> 8) << 16) | ((uint32_t)(uint8_t)(v[3] >> 8) << 24);
}
__device__ __forceinline__ uint32_t pack_lo(const int16_t* v) {   // 4 low bytes, top bit flipped
    return ((uint32_t)(uint8_t)v[0] | ((uint32_t)(uint8_t)v[1] << 8) |
            ((uint32_t)(uint8_t)v[2] << 16) | ((uint32_t)(uint8_t)v[3] << 24)) ^ 0x80808080u;
}

// ---------------------------------------------------------------- operand sources
// A side: rows of the output (matmul rows of A; conv output channels = weights).
struct SrcRowMajor {             // A[i][kk] = a[i * lda + kk]
    const int16_t* p;
    uint32_t rows, k;
    uint64_t lda;
    __device__ bool real(uint32_t i, uint32_t kk) const { return i < rows && kk < k; }
    __device__ int16_t at(uint32_t i, uint32_t kk) const { return p[i * lda + kk]; }
};
// B side: columns of the output; B(kk, j) for the three matmul images.
struct SrcMatB {
    const int16_t* p;
    uint32_t cols, k, m, layout, kw;   // layout 0 row-major, 1 packed, 2 gemv, 3 transposed [m][k]
    __device__ bool real(uint32_t j, uint32_t kk) const { return j < cols && kk < k; }
    __device__ int16_t at(uint32_t j, uint32_t kk) const {
        if (layout == 1) return p[((uint64_t)(j >> 5) * k + kk) * 32 + (j & 31)];
        if (layout == 3) return p[(uint64_t)j * k + kk];
        if (layout == 2 && kw > 1) {
            uint32_t c = (kk / (16 * kw)) * 16 + (kk & 15), jj = (kk >> 4) % kw;
            return p[((uint64_t)c * m + j) * kw + jj];
        }
        return p[(uint64_t)kk * m + j];
    }
};
// Conv weights in the packed tile-major layout (ConvKernel.h:136-159) as GEMM rows:
// kk = ((ict * kh + khi) * kw + kwi) * 16 + lane; lanes past in_ch are padding.
struct SrcConvW {
    const int16_t* p;
    uint32_t out_ch, in_ch, kh, kw, tiles, per_m, last_lanes;
    __device__ bool real(uint32_t mo, uint32_t kk) const {
        uint32_t lane = kk & 15, t = kk >> 4, ict = t / (kh * kw);
        return mo < out_ch && ict < tiles && ict * 16 + lane < in_ch;
    }
    __device__ int16_t at(uint32_t mo, uint32_t kk) const {
        uint32_t lane = kk & 15, t = kk >> 4, ict = t / (kh * kw), pos = t - ict * kh * kw;
        uint32_t lanes = ict + 1 == tiles ? last_lanes : 16;
        return p[(uint64_t)mo * per_m + (uint64_t)ict * kh * kw * 16 + pos * lanes + lane];
    }
};
// im2col of one NCHW image as GEMM columns: column p = oh * out_w + ow.
struct SrcIm2col {
    const int16_t* p;
    uint32_t in_ch, in_h, in_w, out_w, kh, kw, sh, sw, dh, dw, pt, pl, cols;
    __device__ bool real(uint32_t col, uint32_t kk) const {
        uint32_t lane = kk & 15, ict = (kk >> 4) / (kh * kw);
        return col < cols && ict * 16 + lane < in_ch;
    }
    __device__ int16_t at(uint32_t col, uint32_t kk) const {
        uint32_t lane = kk & 15, t = kk >> 4, ict = t / (kh * kw), pos = t - ict * kh * kw;
        uint32_t khi = pos / kw, kwi = pos - khi * kw, ic = ict * 16 + lane;
        uint32_t oh = col / out_w, ow = col - oh * out_w;
        int ih = (int)(oh * sh + khi * dh) - (int)pt, iw = (int)(ow * sw + kwi * dw) - (int)pl;
        if (ih < 0 || ih >= (int)in_h || iw < 0 || iw >= (int)in_w) return 0;
        return p[((uint64_t)ic * in_h + ih) * in_w + iw];
    }
};

// Split one operand into byte planes [lines][kp] (lines = rows for A, columns for B) and
// partial line sums per SLAB of k.  Workgroup: 64 lines x one SLAB; the 64x64 element tiles
// pass through LDS so that the reads follow the source's fast dimension (`KFast`: k for a
// row-major A; the line index for B images and im2col).
template <class Src, bool KFast>
__global__ __launch_bounds__(256) void split_kernel(Src src, uint64_t src_slice, int8_t* __restrict__ hi,
                                                    int8_t* __restrict__ lo, int32_t* __restrict__ part,
                                                    uint32_t lines_p, uint32_t kp, uint32_t nslab) {
    __shared__ int16_t tile[64][64 + 2];
    __shared__ uint8_t realt[64][64 + 4];
    const uint32_t l0 = blockIdx.x * 64, slab = blockIdx.y, bt = blockIdx.z;
    Src s = src;
    s.p = src.p + bt * src_slice;
    const uint64_t pl = (uint64_t)bt * lines_p * kp;
    const uint32_t t = threadIdx.x;
    const uint32_t my_line = t >> 2, part_k = (t & 3) * 16;
    int32_t sum = 0;
    const uint32_t k_end = min(kp, (slab + 1) * SLAB);
    for (uint32_t k0 = slab * SLAB; k0 < k_end; k0 += 64) {
        for (uint32_t r = 0; r < 16; r++) {
            uint32_t idx = r * 256 + t, a, b;
            if (KFast) { a = idx >> 6; b = idx & 63; }       // a = line, b = k
            else { b = idx >> 6; a = idx & 63; }             // b = k, a = line
            bool re = s.real(l0 + a, k0 + b);
            tile[a][b] = re ? s.at(l0 + a, k0 + b) : (int16_t)0;
            realt[a][b] = re;
        }
        __syncthreads();
        int16_t v[16];
        uint32_t hw[4], lw[4];
        for (int q = 0; q < 16; q++) {
            v[q] = tile[my_line][part_k + q];
            if (realt[my_line][part_k + q]) sum += v[q];
        }
        for (int q = 0; q < 4; q++) {
            hw[q] = pack_hi(v + 4 * q);
            lw[q] = pack_lo(v + 4 * q);
            // padding is the byte pair (0, 0)
            for (int e = 0; e < 4; e++)
                if (!realt[my_line][part_k + 4 * q + e]) {
                    hw[q] &= ~(0xFFu << (8 * e));
                    lw[q] &= ~(0xFFu << (8 * e));
                }
        }
        const uint64_t off = pl + (uint64_t)(l0 + my_line) * kp + k0 + part_k;
        *reinterpret_cast<uint4*>(hi + off) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        *reinterpret_cast<uint4*>(lo + off) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
        __syncthreads();
    }
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    if ((t & 3) == 0) part[((uint64_t)bt * nslab + slab) * lines_p + l0 + my_line] = sum;
}

// ---------------------------------------------------------------- bandwidth split kernels
// Padding is written as the value 128 (A' = 0: the byte pair (0, 0)) and left out of the sums.
constexpr int16_t kPad = 128;

// Rows with k contiguous (the matmul A, row stride lda, 16-byte aligned rows): one wavefront
// per row and SLAB of k, 8 k per lane per 16-byte load, the slab's loads all in flight
// before the first is used; grid (ceil(lines_p / 4), nslab, slices).
__global__ __launch_bounds__(256) void split_rows_kernel(const int16_t* __restrict__ src, Slices slice,
                                                         uint64_t lda, uint32_t rows, uint32_t k,
                                                         int8_t* __restrict__ hi, int8_t* __restrict__ lo,
                                                         int32_t* __restrict__ part, uint32_t lines_p,
                                                         uint32_t kp, uint32_t nslab) {
    constexpr int U = SLAB / 512;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6), slab = blockIdx.y, bt = blockIdx.z;
    if (row >= lines_p) return;
    const int16_t* r = src + slice.off(bt) + (uint64_t)row * lda;
    const uint64_t po = ((uint64_t)bt * lines_p + row) * kp;
    const bool real_row = row < rows;
    int4 v[U];
    if (real_row && (slab + 1) * SLAB <= k) {          // the whole slab is real: no branches
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = *reinterpret_cast<const int4*>(r + slab * SLAB + 512 * u + 8 * lane);
    } else {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint32_t k0 = slab * SLAB + 512 * u + 8 * lane;
            int16_t e[8];
#pragma unroll
            for (int q = 0; q < 8; q++) e[q] = (real_row && k0 + q < k) ? r[k0 + q] : kPad;
            v[u] = *reinterpret_cast<const int4*>(e);
        }
    }
    int32_t sum = 0;
#pragma unroll
    for (int u = 0; u < U; u++) {
        const uint32_t k0 = slab * SLAB + 512 * u + 8 * lane;
        if (k0 >= kp) continue;
        if (real_row && k0 + 8 <= k) {
            sum += sum8(v[u]);
        } else {
            const int16_t* e = reinterpret_cast<const int16_t*>(&v[u]);
#pragma unroll
            for (int q = 0; q < 8; q++)
                if (real_row && k0 + q < k) sum += e[q];
        }
        uint2 h, l;
        split8(v[u], h, l);
        *reinterpret_cast<uint2*>(hi + po + k0) = h;
        *reinterpret_cast<uint2*>(lo + po + k0) = l;
    }
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    if (lane == 0) part[((uint64_t)bt * nslab + slab) * lines_p + row] = sum;
}

// Rows of at most 256 k (kp in {64, 128, 192, 256}: one slab): G lanes per row (kp / 8, and 32
// for kp 192 with the last 8 idle), one 16-byte load each, 64 / G rows per wavefront, the row
// sum over the row's lane group.
// Grid (ceil(lines_p / (4 * 64 / G)), 1, slices).
template <uint32_t G>
__global__ __launch_bounds__(256) void split_rows_short_kernel(const int16_t* __restrict__ src, Slices slice,
                                                               uint64_t lda, uint32_t rows, uint32_t k,
                                                               int8_t* __restrict__ hi, int8_t* __restrict__ lo,
                                                               int32_t* __restrict__ part, uint32_t lines_p,
                                                               uint32_t kp) {
    constexpr uint32_t RPW = 64 / G;                       // rows per wavefront
    const uint32_t lane = threadIdx.x & 63, g = lane % G;
    const uint32_t row = (blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW + lane / G, bt = blockIdx.z;
    const uint32_t k0 = 8 * g;
    const bool in = row < lines_p && k0 < kp, real_row = row < rows;
    int4 v = make_int4(0, 0, 0, 0);
    int32_t sum = 0;
    if (in) {
        const int16_t* r = src + slice.off(bt) + (uint64_t)row * lda;
        if (real_row && k0 + 8 <= k) {
            v = *reinterpret_cast<const int4*>(r + k0);
            sum = sum8(v);
        } else {
            int16_t e[8];
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const bool re = real_row && k0 + q < k;
                e[q] = re ? r[k0 + q] : kPad;
                sum += re ? e[q] : 0;
            }
            v = *reinterpret_cast<const int4*>(e);
        }
    }
#pragma unroll
    for (uint32_t off = 1; off < G; off <<= 1) sum += __shfl_xor(sum, off, 64);
    if (!in) return;
    uint2 h, l;
    split8(v, h, l);
    const uint64_t po = ((uint64_t)bt * lines_p + row) * kp + k0;
    *reinterpret_cast<uint2*>(hi + po) = h;
    *reinterpret_cast<uint2*>(lo + po) = l;
    if (g == 0) part[(uint64_t)bt * lines_p + row] = sum;
}

// Columns of a k-major image (row-major B [k][m] with m % 8 == 0, or the packed 32-column
// tiles).  A wavefront takes 32 columns and 256 k of one SLAB: lane = (r4, c8) with
// r4 = lane / 4 picking 4 consecutive k of each 64-k group and c8 = lane % 4 picking 8
// columns, so one load instruction reads 16 rows x 64 contiguous bytes.  Each lane loads
// its 4 groups x 4 rows x 8 columns at once, then transposes every 4 x 8 block in registers
// (byte permutes) into one dword of 4 k per column and plane.  A workgroup is the four
// 256-k quarters of one slab; their column sums meet in LDS.  Grid (ceil(lines_p / 32),
// nslab, slices).
__global__ __launch_bounds__(256) void split_cols_kernel(const int16_t* __restrict__ src, Slices slice,
                                                         uint64_t ldb, uint32_t packed, uint32_t m, uint32_t k,
                                                         int8_t* __restrict__ hi, int8_t* __restrict__ lo,
                                                         int32_t* __restrict__ part, uint32_t lines_p,
                                                         uint32_t kp, uint32_t nslab) {
    __shared__ int32_t csum[4][32];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t r4 = lane >> 2, c8 = lane & 3;
    const uint32_t jg = blockIdx.x * 32, slab = blockIdx.y, bt = blockIdx.z;
    const uint32_t j0 = jg + 8 * c8;                       // this lane's first column
    const int16_t* b = src + slice.off(bt);
    const uint32_t kq = slab * SLAB + 256 * wave;          // this wave's first k
    const bool cols_real = j0 + 8 <= m;
    // element (kk, j) of the image
    auto at = [&](uint32_t kk, uint32_t j) -> uint64_t {
        return packed ? ((uint64_t)(j >> 5) * k + kk) * 32 + (j & 31) : (uint64_t)kk * ldb + j;
    };
    int4 v[4][4];
    if (cols_real && kq + 256 <= k) {                  // every load is real: no branches
        const int16_t* p0 = b + at(kq + 4 * r4, j0);
        const uint64_t rs = packed ? 32 : ldb;         // elements per k row
#pragma unroll
        for (int g = 0; g < 4; g++)
#pragma unroll
            for (int r = 0; r < 4; r++) v[g][r] = *reinterpret_cast<const int4*>(p0 + (64 * g + r) * rs);
    } else {
#pragma unroll
        for (int g = 0; g < 4; g++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t kk = kq + 64 * g + 4 * r4 + r;
                int16_t e[8];
#pragma unroll
                for (int q = 0; q < 8; q++) e[q] = (kk < k && j0 + q < m) ? b[at(kk, j0 + q)] : kPad;
                v[g][r] = *reinterpret_cast<const int4*>(e);
            }
    }
    int32_t sum[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const uint32_t k0 = kq + 64 * g + 4 * r4;
        if (k0 >= kp) continue;
        uint32_t d[4][4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            d[r][0] = (uint32_t)v[g][r].x; d[r][1] = (uint32_t)v[g][r].y;
            d[r][2] = (uint32_t)v[g][r].z; d[r][3] = (uint32_t)v[g][r].w;
            if (k0 + r < k) {
                const int16_t* e = reinterpret_cast<const int16_t*>(&v[g][r]);
#pragma unroll
                for (int q = 0; q < 8; q++)
                    if (j0 + q < m) sum[q] += e[q];
            }
        }
#pragma unroll
        for (int c2 = 0; c2 < 4; c2++) {               // columns 2 c2 and 2 c2 + 1
            const uint32_t xh = __builtin_amdgcn_perm(d[1][c2], d[0][c2], 0x07030501u);
            const uint32_t yh = __builtin_amdgcn_perm(d[3][c2], d[2][c2], 0x07030501u);
            const uint32_t xl = __builtin_amdgcn_perm(d[1][c2], d[0][c2], 0x06020400u);
            const uint32_t yl = __builtin_amdgcn_perm(d[3][c2], d[2][c2], 0x06020400u);
            const uint64_t o0 = ((uint64_t)bt * lines_p + j0 + 2 * c2) * kp + k0;
            const uint64_t o1 = o0 + kp;
            *reinterpret_cast<uint32_t*>(hi + o0) = __builtin_amdgcn_perm(yh, xh, 0x05040100u);
            *reinterpret_cast<uint32_t*>(hi + o1) = __builtin_amdgcn_perm(yh, xh, 0x07060302u);
            *reinterpret_cast<uint32_t*>(lo + o0) = __builtin_amdgcn_perm(yl, xl, 0x05040100u) ^ 0x80808080u;
            *reinterpret_cast<uint32_t*>(lo + o1) = __builtin_amdgcn_perm(yl, xl, 0x07060302u) ^ 0x80808080u;
        }
    }
    // column sums: over the 16 lanes of one c8 (lane bits 2..5), then the four waves
#pragma unroll
    for (int q = 0; q < 8; q++) {
        int32_t x = sum[q];
        for (int off = 4; off < 64; off <<= 1) x += __shfl_xor(x, off, 64);
        sum[q] = x;
    }
    if (r4 == 0) {
#pragma unroll
        for (int q = 0; q < 8; q++) csum[wave][8 * c8 + q] = sum[q];
    }
    __syncthreads();
    if (threadIdx.x < 32 && jg + threadIdx.x < lines_p)
        part[((uint64_t)bt * nslab + slab) * lines_p + jg + threadIdx.x] =
            csum[0][threadIdx.x] + csum[1][threadIdx.x] + csum[2][threadIdx.x] + csum[3][threadIdx.x];
}

// 1x1 stride-1 convolutions with the images folded into the GEMM's columns: line
// j = img * plane + p is pixel p of image img, k the input channel, B(c, j) = x[img][c][p].
// For planes that are not a multiple of 8 pixels.  A workgroup takes 64 lines and one SLAB
// of k, each of its waves (up to 16) 64 k in 16-k chunks: lane = line, 16 loads of 2 bytes
// (the 64 lanes of one load read 128 consecutive bytes of one channel row where the lines
// stay in one image), packed into one 16-byte word per plane.  Grid (lines_p / 64, nslab).
__global__ __launch_bounds__(1024) void split_fold_kernel(const int16_t* __restrict__ x, uint32_t in_ch,
                                                          uint32_t plane, uint64_t img_elems, uint32_t cols,
                                                          int8_t* __restrict__ hi, int8_t* __restrict__ lo,
                                                          int32_t* __restrict__ part, uint32_t lines_p, uint32_t kp) {
    __shared__ int32_t wsum[16][64];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    const uint32_t j = blockIdx.x * 64 + lane, slab = blockIdx.y;
    const bool real = j < cols;
    const uint32_t img = real ? j / plane : 0, p = real ? j - img * plane : 0;
    const int16_t* src = x + img * img_elems + p;
    int32_t sum = 0;
    const uint32_t kb = slab * SLAB + 64 * wave, ke = min(kb + 64, kp);
    // the wave's four 16-k chunks unrolled: every load in flight before the first is used
#pragma unroll 4
    for (uint32_t k0 = kb; k0 < ke; k0 += 16) {
        int16_t e[16];
        if (real && k0 + 16 <= in_ch) {
#pragma unroll
            for (int q = 0; q < 16; q++) e[q] = src[(uint64_t)(k0 + q) * plane];
#pragma unroll
            for (int q = 0; q < 16; q++) sum += e[q];
        } else {
#pragma unroll
            for (int q = 0; q < 16; q++) {
                const bool r = real && k0 + q < in_ch;
                e[q] = r ? src[(uint64_t)(k0 + q) * plane] : kPad;
                sum += r ? e[q] : 0;
            }
        }
        uint2 h0, l0, h1, l1;
        split8(*reinterpret_cast<const int4*>(e), h0, l0);
        split8(*reinterpret_cast<const int4*>(e + 8), h1, l1);
        const uint64_t off = (uint64_t)j * kp + k0;
        *reinterpret_cast<uint4*>(hi + off) = make_uint4(h0.x, h0.y, h1.x, h1.y);
        *reinterpret_cast<uint4*>(lo + off) = make_uint4(l0.x, l0.y, l1.x, l1.y);
    }
    wsum[wave][lane] = sum;
    __syncthreads();
    if (wave == 0) {
        int32_t t = 0;
        for (uint32_t w = 0; w < waves; w++) t += wsum[w][lane];
        part[(uint64_t)slab * lines_p + j] = t;
    }
}

// The same operand for few lines (small planes): 16 lines a workgroup so that the grid has
// four times the workgroups.  Wave w takes the slab's 64 k from 64 w; lane (line l % 16, chunk
// l / 16) loads its line's 16 k of the chunk (the 16 lanes of one chunk read 32 consecutive bytes
// of a channel row where the lines stay in one image), so the four chunk lanes of a line write
// 64 contiguous bytes of each plane.  Grid (lines_p / 16, nslab).
__global__ __launch_bounds__(1024) void split_fold16_kernel(const int16_t* __restrict__ x, uint32_t in_ch,
                                                            uint32_t plane, uint64_t img_elems, uint32_t cols,
                                                            int8_t* __restrict__ hi, int8_t* __restrict__ lo,
                                                            int32_t* __restrict__ part, uint32_t lines_p,
                                                            uint32_t kp) {
    __shared__ int32_t wsum[16][16];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    const uint32_t ln = lane & 15, ch = lane >> 4;
    const uint32_t j = blockIdx.x * 16 + ln, slab = blockIdx.y;
    const bool real = j < cols;
    const uint32_t img = real ? j / plane : 0, p = real ? j - img * plane : 0;
    const int16_t* src = x + img * img_elems + p;
    int32_t sum = 0;
    const uint32_t k0 = slab * SLAB + 64 * wave + 16 * ch;
    if (k0 < kp) {
        int16_t e[16];
        if (real && k0 + 16 <= in_ch) {
#pragma unroll
            for (int q = 0; q < 16; q++) e[q] = src[(uint64_t)(k0 + q) * plane];
#pragma unroll
            for (int q = 0; q < 16; q++) sum += e[q];
        } else {
#pragma unroll
            for (int q = 0; q < 16; q++) {
                const bool r = real && k0 + q < in_ch;
                e[q] = r ? src[(uint64_t)(k0 + q) * plane] : kPad;
                sum += r ? e[q] : 0;
            }
        }
        uint2 h0, l0, h1, l1;
        split8(*reinterpret_cast<const int4*>(e), h0, l0);
        split8(*reinterpret_cast<const int4*>(e + 8), h1, l1);
        const uint64_t off = (uint64_t)j * kp + k0;
        *reinterpret_cast<uint4*>(hi + off) = make_uint4(h0.x, h0.y, h1.x, h1.y);
        *reinterpret_cast<uint4*>(lo + off) = make_uint4(l0.x, l0.y, l1.x, l1.y);
    }
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    if (ch == 0) wsum[wave][ln] = sum;
    __syncthreads();
    if (threadIdx.x < 16) {
        int32_t t = 0;
        for (uint32_t w = 0; w < waves; w++) t += wsum[w][threadIdx.x];
        part[(uint64_t)slab * lines_p + blockIdx.x * 16 + threadIdx.x] = t;
    }
}

// The same operand for planes with many lines: a workgroup takes 64 lines and one SLAB of
// k in 64 x 64 tiles through LDS.  Thread t loads line t % 64 at 16 k (2-byte loads, the 64
// lanes of one load on consecutive lines), then packs 16 consecutive k of line t / 4 into
// 16-byte words: the four threads of a line write 64 contiguous bytes of each plane.
// Grid (lines_p / 64, nslab).
__global__ __launch_bounds__(256) void split_fold_lds_kernel(const int16_t* __restrict__ x, uint32_t in_ch,
                                                             uint32_t plane, uint64_t img_elems, uint32_t cols,
                                                             int8_t* __restrict__ hi, int8_t* __restrict__ lo,
                                                             int32_t* __restrict__ part, uint32_t lines_p,
                                                             uint32_t kp) {
    __shared__ int16_t tile[64][64 + 2];
    const uint32_t t = threadIdx.x, la = t & 63, kr = t >> 6;
    const uint32_t l0 = blockIdx.x * 64, slab = blockIdx.y;
    const uint32_t ja = l0 + la;
    const bool real_a = ja < cols;
    const uint32_t img = real_a ? ja / plane : 0, pa = real_a ? ja - img * plane : 0;
    const int16_t* src = x + img * img_elems + pa;
    const uint32_t my_line = t >> 2, part_k = (t & 3) * 16;
    int32_t sum = 0;
    const uint32_t k_end = min(kp, (slab + 1) * SLAB);
    // a 64-k chunk's loads in registers, the next chunk's issued while this one is split
    int16_t v[16];
    auto load_chunk = [&](uint32_t k0) {
#pragma unroll
        for (uint32_t r = 0; r < 16; r++) {
            const uint32_t kk = k0 + 4 * r + kr;
            v[r] = (real_a && kk < in_ch) ? src[(uint64_t)kk * plane] : kPad;
        }
    };
    load_chunk(slab * SLAB);
    for (uint32_t k0 = slab * SLAB; k0 < k_end; k0 += 64) {
#pragma unroll
        for (uint32_t r = 0; r < 16; r++) tile[la][4 * r + kr] = v[r];
        __syncthreads();
        if (k0 + 64 < k_end) load_chunk(k0 + 64);
        int16_t e[16];
#pragma unroll
        for (int q = 0; q < 16; q++) {
            e[q] = tile[my_line][part_k + q];
            sum += (l0 + my_line < cols && k0 + part_k + q < in_ch) ? e[q] : 0;
        }
        uint2 h0, lw0, h1, lw1;
        split8(*reinterpret_cast<const int4*>(e), h0, lw0);
        split8(*reinterpret_cast<const int4*>(e + 8), h1, lw1);
        const uint64_t off = (uint64_t)(l0 + my_line) * kp + k0 + part_k;
        *reinterpret_cast<uint4*>(hi + off) = make_uint4(h0.x, h0.y, h1.x, h1.y);
        *reinterpret_cast<uint4*>(lo + off) = make_uint4(lw0.x, lw0.y, lw1.x, lw1.y);
        __syncthreads();
    }
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    if ((t & 3) == 0) part[(uint64_t)slab * lines_p + l0 + my_line] = sum;
}

// ---------------------------------------------------------------- epilogues
// An epilogue names where output row `i` of slice `bt` starts (nullptr past the last row),
// the raw per-row bias (added to the sum as bias << 8), the offset of column `j` from a row
// start, and whether every row start and the column count are even (then two adjacent
// results go out as one 4-byte store).
struct TileBase {               // a tile's first output element and row stride (nullptr: none)
    int16_t* base;
    uint32_t ld;
};
struct EpiMatmul {              // C[bt][i][j] = c + off(bt) + i * ldc + j
    int16_t* c;
    uint64_t c_bs;
    uint32_t rows, cols, wrap, pairs;
    uint64_t ldc = 0;           // row stride (0: cols)
    uint64_t c_bs2 = 0;         // with `inner` > 1: slice bt at (bt / inner) c_bs + (bt % inner) c_bs2
    uint32_t inner = 1;
    int32_t lo = -32768, hi = 32767;    // output bounds (the saturation; a fused RELU / RELU6 narrows them)
    __device__ int32_t row_bias(uint32_t) const { return 0; }
    __device__ int16_t* row_ptr(uint32_t bt, uint32_t i) const {
        if (i >= rows) return nullptr;
        const uint64_t off = inner > 1 ? (uint64_t)(bt / inner) * c_bs + (uint64_t)(bt % inner) * c_bs2 : bt * c_bs;
        return c + off + (uint64_t)i * (ldc ? ldc : cols);
    }
    __device__ uint64_t col_off(uint32_t j) const { return j; }
    // The tile (row0, col0) of tm x tn wholly inside C with paired stores: its first element
    // and the row stride, so that element (r, c) of the tile sits at base + r * ld + c.
    __device__ __forceinline__ TileBase tile_base(uint32_t bt, uint32_t row0, uint32_t col0, uint32_t tm,
                                                  uint32_t tn) const {
        const uint64_t l = ldc ? ldc : cols;
        if (!pairs || row0 + tm > rows || col0 + tn > cols || l * tm >= (1ull << 30)) return TileBase{nullptr, 0};
        return TileBase{row_ptr(bt, row0) + col0, (uint32_t)l};
    }
};
struct EpiConv {                // y pattern (ConvKernel.h:250-258); acc seeded with bias << 8
    int16_t* y;
    const int16_t* bias;
    uint64_t img;               // elements per image (out_ch * plane)
    uint32_t rows, cols, cs, cn, gs, wrap, pairs;
    uint32_t fold;              // pixels per image when the images are folded into the columns, else 0
    int32_t lo = -32768, hi = 32767;    // output bounds (the saturation; a fused RELU / RELU6 narrows them)
    __device__ int32_t row_bias(uint32_t i) const { return bias && i < rows ? (int32_t)bias[i] : 0; }
    __device__ int16_t* row_ptr(uint32_t bt, uint32_t i) const {
        if (i >= rows) return nullptr;
        const uint64_t base = cn ? (uint64_t)(i % cn) * cs + (uint64_t)(i / cn) * gs : (uint64_t)i * cs;
        return y + bt * img + base;
    }
    __device__ uint64_t col_off(uint32_t j) const {
        if (!fold) return j;
        const uint32_t im = j / fold;
        return (uint64_t)im * img + (j - im * fold);
    }
    __device__ __forceinline__ TileBase tile_base(uint32_t bt, uint32_t row0, uint32_t col0, uint32_t tm,
                                                  uint32_t tn) const {
        if (!pairs || fold || cn || row0 + tm > rows || col0 + tn > cols || (uint64_t)cs * tm >= (1ull << 30))
            return TileBase{nullptr, 0};
        return TileBase{row_ptr(bt, row0) + col0, cs};
    }
};

// Recombination modes of the output rule floor(acc / 2^8) -> int16:
//   acc = 2^16 HH + 2^8 MID + LL + 128 rowsum + 128 colsum - 16384 K + 2^8 bias.
// With rowsum = 2 rh' + rl', colsum likewise (arithmetic shift, low bit),
//   floor(acc / 2^8) = 2^8 HH + MID + rh + ch + ((LL + rl + cl) >> 8),
//   rh = bias - 64 K + (rowsum >> 1), rl = 128 (rowsum & 1), ch = colsum >> 1, cl = 128 (colsum & 1),
// every term but 2^8 HH exact in int32 for K <= 32768.
//   kSatNarrow (K <= 8192): |the rest| < 2^29.1, so clamping HH to +-2^22 keeps the sum in
//     int32 and cannot change a saturated result (|2^8 HH| > 2^30 then decides the sign);
//   kWrap: the sum wrapped to int32 first, i.e. floor(acc / 2^8) mod 2^24, sign-extended;
//   kSatWide (K > 8192, saturating): the sum in int64.
//   kSplitFix (wrap products split over k): every slice stores its 2^16 HH + 2^8 MID + LL
//     mod 2^32 as int32 partials, and the slice of a tile that arrives last adds the others'
//     to its own and stores the tile by the kWrap rule (split_fixup).
enum : uint32_t { kSatNarrow = 0, kWrap = 1, kSatWide = 2, kSplitFix = 3 };

__device__ __forceinline__ int32_t clamp_i32(int32_t v, int32_t lo, int32_t hi) {   // v_med3_i32
    return min(max(v, lo), hi);
}

// The result is clamped to [lo, hi] inside the int16 range: the saturation, or with a fused
// RELU (lo = 0) / RELU6 (lo = 0, hi = 6 * 2^8) the activation of the saturated value as well.
template <uint32_t MODE>
__device__ __forceinline__ int32_t recombine(int32_t hh, int32_t mid, int32_t ll, int32_t rhch, int32_t rlcl,
                                             int32_t lo, int32_t hi) {
    const int32_t y = mid + rhch + ((ll + rlcl) >> 8);
    int32_t q;
    if (MODE == kSatNarrow) {
        q = (int32_t)((uint32_t)clamp_i32(hh, -(1 << 22), 1 << 22) << 8) + y;
    } else if (MODE == kWrap) {
        q = (int32_t)(((uint32_t)hh << 8) + (uint32_t)y);
        q = (q << 8) >> 8;
    } else {
        const long long w = ((long long)hh << 8) + (long long)mid + (long long)rhch + ((ll + rlcl) >> 8);
        q = (int32_t)(w > 32767 ? 32767 : (w < -32768 ? -32768 : w));
    }
    return clamp_i32(q, lo, hi);
}

typedef int v16i __attribute__((ext_vector_type(16)));

// Store one wave's 64 x 64 results.  A lane holds D[8 (r / 4) + 4 lh + r % 4][l32] of each
// 32 x 32 block.  With PAIRS, lanes 2c and 2c + 1 swap one result per row pair (DPP
// quad_perm [1,0,3,2]) so that the even lane stores columns (2c, 2c + 1) of row r and the
// odd lane the same columns of row r + 1, as one 4-byte store each.
template <uint32_t MODE, bool PAIRS, class Epi>
__device__ __forceinline__ void store_wave_tile(const v16i (&hh)[2][2], const v16i (&mid)[2][2],
                                                const v16i (&ll)[2][2], const int2* rterm, const int2* cterm,
                                                uint32_t bt, uint32_t row0, uint32_t col0, uint32_t wr,
                                                uint32_t wc, uint32_t l32, uint32_t lh, const Epi& epi) {
    const uint32_t odd = l32 & 1;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const uint32_t cl = wc * 64 + j * 32 + l32, col = col0 + cl;
        const int2 ct = cterm[cl];
#pragma unroll
        for (int i = 0; i < 2; i++) {
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                const uint32_t rl = wr * 64 + i * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                const int2 r0 = rterm[rl], r1 = rterm[rl + 1];
                const int32_t q0 = recombine<MODE>(hh[i][j][r], mid[i][j][r], ll[i][j][r], r0.x + ct.x, r0.y + ct.y,
                                                   epi.lo, epi.hi);
                const int32_t q1 = recombine<MODE>(hh[i][j][r + 1], mid[i][j][r + 1], ll[i][j][r + 1], r1.x + ct.x,
                                                   r1.y + ct.y, epi.lo, epi.hi);
                if (PAIRS) {
                    const int32_t give = odd ? q0 : q1;
                    const int32_t got = __builtin_amdgcn_mov_dpp(give, 0xB1, 0xF, 0xF, false);
                    const uint32_t lo = (uint32_t)(odd ? got : q0) & 0xFFFFu;
                    const uint32_t hi = (uint32_t)(odd ? q1 : got) << 16;
                    int16_t* dst = epi.row_ptr(bt, row0 + rl + odd);
                    if (dst != nullptr && col - odd < epi.cols)
                        *reinterpret_cast<uint32_t*>(dst + epi.col_off(col - odd)) = lo | hi;
                } else if (col < epi.cols) {
                    int16_t* d0 = epi.row_ptr(bt, row0 + rl);
                    int16_t* d1 = epi.row_ptr(bt, row0 + rl + 1);
                    const uint64_t co = epi.col_off(col);
                    if (d0 != nullptr) d0[co] = (int16_t)q0;
                    if (d1 != nullptr) d1[co] = (int16_t)q1;
                }
                // one row pair at a time: hoisting the term loads of later pairs would
                // need more registers than the accumulators leave
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
}

// store_wave_tile for a tile wholly inside the output with plain rows (tile_base): the lane's
// offset from the tile's first element in 32 bits, the row offsets uniform, no bounds checks.
template <uint32_t MODE>
__device__ __forceinline__ void store_wave_fast(const v16i (&hh)[2][2], const v16i (&mid)[2][2],
                                                const v16i (&ll)[2][2], const int2* rterm, const int2* cterm,
                                                int16_t* __restrict__ base, uint32_t ld, uint32_t wr, uint32_t wc,
                                                uint32_t l32, uint32_t lh, int32_t lo, int32_t hi) {
    const uint32_t odd = l32 & 1;
    const uint32_t lane_off = (wr * 64 + 4 * lh + odd) * ld + wc * 64 + l32 - odd;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int2 ct = cterm[wc * 64 + j * 32 + l32];
#pragma unroll
        for (int i = 0; i < 2; i++) {
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                const uint32_t rl = wr * 64 + i * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                const int2 r0 = rterm[rl], r1 = rterm[rl + 1];
                const int32_t q0 = recombine<MODE>(hh[i][j][r], mid[i][j][r], ll[i][j][r], r0.x + ct.x, r0.y + ct.y,
                                                   lo, hi);
                const int32_t q1 = recombine<MODE>(hh[i][j][r + 1], mid[i][j][r + 1], ll[i][j][r + 1], r1.x + ct.x,
                                                   r1.y + ct.y, lo, hi);
                // the pair exchange of store_wave_tile: the even lane stores row r, the odd lane row r + 1
                const int32_t give = odd ? q0 : q1;
                const int32_t got = __builtin_amdgcn_mov_dpp(give, 0xB1, 0xF, 0xF, false);
                const uint32_t lo = (uint32_t)(odd ? got : q0), hi = (uint32_t)(odd ? q1 : got);
                const uint32_t roff = (uint32_t)(i * 32 + 8 * (r >> 2) + (r & 3)) * ld + j * 32;
                *reinterpret_cast<uint32_t*>(base + lane_off + roff) = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
}

// kSplitFix: this slice's partial of its wave's 64 x 64 outputs, in the accumulators' own
// layout (a tile's nz slices are consecutive blocks of TM x 128 int32 at `tile_part`; in a
// block, wave w's accumulator (i, j) rows 4q .. 4q + 3 sit at 1 KiB row (4 (2i + j) + q) of
// the wave's 16 KiB, 16 bytes a lane), written and read with agent-scope 16-byte buffer
// accesses (sc1) so that a workgroup on another XCD reads them; then the tile's arrival count.
// The slice that arrives last (ticket nz - 1) resets the count for the next launch, adds the
// other slices' partials (all were stored, and their stores had completed, before their slices
// took their tickets) and returns true with the wrapped total T in limb form -- HH = T >> 16,
// MID = (T >> 8) & 255, LL = T & 255, 2^16 HH + 2^8 MID + LL = T exactly -- for the kWrap
// store; the other slices return false.  No workgroup waits for another.  Every wave of the
// workgroup calls it (two barriers).
template <int TM>
__device__ __forceinline__ bool split_fixup(v16i (&hh)[2][2], v16i (&mid)[2][2], v16i (&ll)[2][2],
                                            int32_t* tile_part, uint32_t nz, uint32_t kz, uint32_t wave,
                                            uint32_t lane, uint32_t* cnt, uint32_t* ticket) {
    constexpr uint32_t kBlock = TM * 128 * 4;                  // bytes of one slice's tile
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(tile_part, 0, (int)(nz * kBlock), 0x00020000);
    const uint32_t wbase = wave * 16384 + lane * 16;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++)
                ll[i][j][r] = (int32_t)(((uint32_t)hh[i][j][r] << 16) + ((uint32_t)mid[i][j][r] << 8) +
                                        (uint32_t)ll[i][j][r]);
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const v4i v = {ll[i][j][4 * q], ll[i][j][4 * q + 1], ll[i][j][4 * q + 2], ll[i][j][4 * q + 3]};
                __builtin_amdgcn_raw_buffer_store_b128(v, rs, kz * kBlock + wbase + (4 * (2 * i + j) + q) * 1024, 0, 16);
            }
    __builtin_amdgcn_s_waitcnt(0x0070);      // this wave's partial stores complete
    __syncthreads();
    if (threadIdx.x == 0) *ticket = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (*ticket != nz - 1) return false;
    if (threadIdx.x == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (uint32_t z = 0; z < nz; z++) {
        if (z == kz) continue;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const v4i v = __builtin_amdgcn_raw_buffer_load_b128(rs, z * kBlock + wbase + (4 * (2 * i + j) + q) * 1024, 0, 16);
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        ll[i][j][4 * q + e] = (int32_t)((uint32_t)ll[i][j][4 * q + e] + (uint32_t)v[e]);
                }
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int32_t tot = ll[i][j][r];
                hh[i][j][r] = tot >> 16;
                mid[i][j][r] = (tot >> 8) & 255;
                ll[i][j][r] = tot & 255;
            }
    return true;
}

// ---------------------------------------------------------------- the plane GEMM
// Grid: x = output tiles of one slice (XCD-aware order), y = batch slice, z = k slice (with
// `ksteps` k steps each; 0: no split).  a_slice /
// b_slice: plane bytes per slice (0 = broadcast); the row / column partial sums per SLAB of
// k sit at part[(slice * nslab + s) * lines + line] (slice stride 0 = broadcast).
//
// A workgroup computes a (64 WR) x 128 tile with 2 WR waves in a WR x 2 arrangement, 64 x 64
// outputs each: 2 x 2 blocks of v_mfma_i32_32x32x32_i8 (the i8 MFMA that sustains the full
// rate on gfx950), three int32 accumulators per block (192 registers), so two waves share
// each SIMD:
//   WR = 4, NST = 3: 8 waves, one workgroup per CU, a three-stage LDS ring (144 KiB) with
//     the copies two steps ahead.  Both waves of a SIMD meet at the same barriers, so
//     neither is starved (with two workgroups per CU the older one takes issue priority and
//     the younger finishes alone, at one wave per SIMD);
//   WR = 2, NST = 2: 4 waves, two workgroups per CU, a two-stage ring (64 KiB), for row
//     counts that do not fill 256-row tiles.
// Step k issues the global -> LDS copies (global_load_lds_dwordx4, no registers) of step
// k + NST - 1 at its top, and ends by waiting for this wave's copies of step k + 1 and its
// fragment reads, then for every wave (barrier).  LDS layout: per stage and plane a
// [rows][64 B] tile; row r holds its 16-byte chunk c at chunk c ^ ((r >> 2) & 3), so any
// 16 consecutive rows of one chunk hit 16 distinct bank groups.  A direct copy writes 1 KiB
// (16 rows) per wave instruction, lane l at 16 l.
__device__ __forceinline__ void lds_copy16(const int8_t* g, int8_t* lds_wave_base) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds_wave_base, 16, 0, 0);
}

template <int WR, int NST, class Epi>
__global__ __launch_bounds__(128 * WR, WR == 1 ? 1 : 8 / (2 * WR)) void gemm_planes_kernel(
    const int8_t* __restrict__ Ahi, const int8_t* __restrict__ Alo, const int32_t* __restrict__ rpart,
    uint64_t a_slice, uint64_t rp_slice, uint32_t a_lines, const int8_t* __restrict__ Bhi,
    const int8_t* __restrict__ Blo, const int32_t* __restrict__ cpart, uint64_t b_slice, uint64_t cp_slice,
    uint32_t b_lines, uint32_t nslab, uint32_t nsum_a, uint32_t tiles_r, uint32_t tiles_c, uint32_t kp, int32_t k64,
    uint32_t mode, int32_t* __restrict__ pout, uint32_t ksteps, uint32_t* __restrict__ tcnt, Epi epi) {
    constexpr int TM = 64 * WR;                  // tile rows
    constexpr int NT = 128 * WR;                 // threads
    constexpr int NW = 2 * WR;                   // waves
    constexpr int A_T = TM * BK, B_T = BN * BK;  // plane tile bytes
    constexpr int STAGE = 2 * A_T + 2 * B_T;     // Ah, Al, Bh, Bl
    constexpr int BCP = 8 / NW;                  // 16-row blocks of a B plane per wave
    constexpr int NC = 2 * 2 + 2 * BCP;          // copies per thread and step
    static_assert(NST == 2 || NST == 3, "two or three stages");
    // the stages as separate arrays: with the loop unrolled by NST every access names its
    // stage statically, so the compiler tells the copies in flight into the other stages
    // from the fragment reads
    __shared__ __attribute__((aligned(1024))) int8_t sm0[STAGE];
    __shared__ __attribute__((aligned(1024))) int8_t sm1[STAGE];
    __shared__ __attribute__((aligned(1024))) int8_t sm2[NST == 3 ? STAGE : 16];
    __shared__ int2 rterm[TM], cterm[BN];        // (h, l) halves
    __shared__ uint32_t ticket;                  // kSplitFix: the tile's arrival ticket

    // XCD-aware tile order: workgroups are dispatched round-robin over the 8 XCDs, so
    // give each XCD a contiguous range of tiles (column-major: tiles sharing a B column
    // strip run on one XCD and share its L2).
    const uint32_t ntiles = tiles_r * tiles_c;
    uint32_t g = blockIdx.x;
    if ((ntiles & 7) == 0) g = (g & 7) * (ntiles >> 3) + (g >> 3);
    const uint32_t tr = g % tiles_r, tc = g / tiles_r;
    const uint32_t bt = blockIdx.y, kz = blockIdx.z;
    const uint32_t kbeg = ksteps ? kz * ksteps : 0;

    const uint32_t t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const uint32_t wr = wave >> 1, wc = wave & 1, l32 = lane & 31, lh = lane >> 5;

    // Row / column terms of the epilogue from the slab partials: the first slab's loads are
    // issued here and used only after the first copies have been issued, so that the two
    // latencies overlap; the other slabs and the LDS writes follow the copies.
    constexpr int TE = (TM + BN + NT - 1) / NT;  // term elements per thread
    int32_t tsum[TE];
#pragma unroll
    for (int q = 0; q < TE; q++) {
        const uint32_t e = t + q * NT;
        tsum[q] = 0;
        if (e < TM + BN)
            tsum[q] = e < TM ? rpart[bt * rp_slice + tr * TM + e] : cpart[bt * cp_slice + tc * BN + (e - TM)];
    }
    auto finish_terms = [&]() {
#pragma unroll
        for (int q = 0; q < TE; q++) {
            const uint32_t e = t + q * NT;
            if (e >= TM + BN) continue;
            const bool is_row = e < TM;
            const uint32_t line = is_row ? tr * TM + e : tc * BN + (e - TM);
            const int32_t* pp = is_row ? rpart + bt * rp_slice + line : cpart + bt * cp_slice + line;
            const uint32_t stride = is_row ? a_lines : b_lines;
            int32_t sum = tsum[q];
            const uint32_t ns = is_row ? nsum_a : nslab;
            for (uint32_t sl = 1; sl < ns; sl++) sum += pp[(uint64_t)sl * stride];
            if (is_row) rterm[e] = make_int2(epi.row_bias(line) - k64 + (sum >> 1), (sum & 1) << 7);
            else cterm[e - TM] = make_int2(sum >> 1, (sum & 1) << 7);
        }
    };

    // copy assignment: wave w fills 16-row blocks 2w, 2w + 1 of each A plane and BCP blocks
    // from BCP w of each B plane; lane l takes row 16 b + l / 4, physical chunk l % 4 =
    // logical chunk (l % 4) ^ swizzle (the swizzle depends on l / 4 only)
    const uint32_t lrow = lane >> 2, cchunk = ((lane & 3) ^ ((lrow >> 2) & 3)) * 16;
    const uint64_t a_base = bt * a_slice + (uint64_t)tr * TM * kp + (uint64_t)kbeg * BK;
    const uint64_t b_base = bt * b_slice + (uint64_t)tc * BN * kp + (uint64_t)kbeg * BK;
    const int8_t* ah_src = Ahi + a_base + (uint64_t)(32 * wave + lrow) * kp + cchunk;
    const int8_t* al_src = Alo + a_base + (uint64_t)(32 * wave + lrow) * kp + cchunk;
    const int8_t* bh_src = Bhi + b_base + (uint64_t)(16 * BCP * wave + lrow) * kp + cchunk;
    const int8_t* bl_src = Blo + b_base + (uint64_t)(16 * BCP * wave + lrow) * kp + cchunk;
    const uint64_t kp16 = (uint64_t)16 * kp;
    const uint32_t a_dst = __builtin_amdgcn_readfirstlane(2048 * wave);
    const uint32_t b_dst = __builtin_amdgcn_readfirstlane(1024 * BCP * wave);

    // fragment read offsets: lane reads row base32 + l32, logical chunk 2 s + lh (substep s)
    const uint32_t sw = (l32 >> 2) & 3;
    const uint32_t fa_row = (wr * 64 + l32) * BK, fb_row = (wc * 64 + l32) * BK;
    const uint32_t ch0 = ((0 + lh) ^ sw) * 16, ch1 = ((2 + lh) ^ sw) * 16;

    v16i hh[2][2], mid[2][2], ll[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) hh[i][j] = mid[i][j] = ll[i][j] = v16i{};
    v4i ah[2], al[2], bh[2], bl[2];

    const uint32_t nk = ksteps ? min(ksteps, kp / BK - kbeg) : kp / BK;
    // Copy group: the two waves sharing a SIMD (w and w + 4 of 8, as dispatched) issue
    // their copies in different substeps.  With 4 waves per workgroup all are group 0.
    const uint32_t cgrp = NW == 8 ? __builtin_amdgcn_readfirstlane((wave >> 2) & 1) : 0;
    // Copy q of a step (0, 1: A hi; 2, 3: A lo; then B hi, B lo); A rows 16 apart, B blocks.
#define CM_COPY(SM, step, q)                                                                        \
    {                                                                                               \
        const uint64_t k_ = (uint64_t)(step) * BK;                                                  \
        if ((q) < 2) lds_copy16(ah_src + (q) * kp16 + k_, &SM[a_dst + 1024 * (q)]);                 \
        else if ((q) < 4) lds_copy16(al_src + ((q) - 2) * kp16 + k_, &SM[A_T + a_dst + 1024 * ((q) - 2)]); \
        else if ((q) < 4 + BCP)                                                                     \
            lds_copy16(bh_src + ((q) - 4) * kp16 + k_, &SM[2 * A_T + b_dst + 1024 * ((q) - 4)]);    \
        else                                                                                        \
            lds_copy16(bl_src + ((q) - 4 - BCP) * kp16 + k_, &SM[2 * A_T + B_T + b_dst + 1024 * ((q) - 4 - BCP)]); \
    }
    // The copies of slot s (after the s-th group of four MFMAs, 0..7): waves of copy group
    // g issue theirs in slots 4g .. 4g + 3, two, two, then the rest; with 2 waves (12 copies)
    // the one group issues two in each of slots 0 .. 5.
#define CM_COPIES(SM, step, slot)                                                 \
    if (!cp_) {                                                                   \
    } else if (NW == 2) {                                                         \
        if ((slot) < 6) { CM_COPY(SM, step, 2 * (slot)) CM_COPY(SM, step, 2 * (slot) + 1) } \
    } else if (((slot) >> 2) == cgrp) {                                           \
        constexpr int s_ = (slot) & 3;                                            \
        if (s_ < 2) { CM_COPY(SM, step, 2 * s_) CM_COPY(SM, step, 2 * s_ + 1) }   \
        else if (NC == 6) { CM_COPY(SM, step, 2 + s_) }                           \
        else { CM_COPY(SM, step, 2 * s_) CM_COPY(SM, step, 2 * s_ + 1) }          \
    }                                                                             \
    __builtin_amdgcn_sched_barrier(0);
#define CM_FRAGS(SM, CH)                                                                   \
    _Pragma("unroll") for (int b = 0; b < 2; b++) {                                        \
        ah[b] = *reinterpret_cast<const v4i*>(&SM[fa_row + b * 32 * BK + CH]);             \
        al[b] = *reinterpret_cast<const v4i*>(&SM[A_T + fa_row + b * 32 * BK + CH]);       \
        bh[b] = *reinterpret_cast<const v4i*>(&SM[2 * A_T + fb_row + b * 32 * BK + CH]);   \
        bl[b] = *reinterpret_cast<const v4i*>(&SM[2 * A_T + B_T + fb_row + b * 32 * BK + CH]); \
    }                                                                                      \
    __builtin_amdgcn_sched_barrier(0);
    // four MFMAs of one limb product over the 2 x 2 blocks
#define CM_MFMA4(ACC, X, Y)                                                                       \
    _Pragma("unroll") for (int i = 0; i < 2; i++) _Pragma("unroll") for (int j = 0; j < 2; j++)   \
        ACC[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(X[i], Y[j], ACC[i][j], 0, 0, 0);       \
    __builtin_amdgcn_sched_barrier(0);
    // One k step on stage SMC while later steps land in the others; SMI receives step
    // kt + NST - 1 when there is one (a wave-uniform branch around each copy).  Two 32-k substeps of 16 MFMAs (hh, mid = h l, ll, mid = l h: no MFMA
    // waits on the one before); the step's copies sit between MFMA groups of the substep
    // of the wave's copy group, so that while one wave of a SIMD spends issue cycles on
    // copies the other has MFMAs to issue, and the sched_barriers keep the compiler from
    // gathering them.  The end of the step waits for this wave's copies of step kt + 1
    // (this step's NC may stay in flight with three stages) and fragment reads, then for
    // every wave.
#define CM_SUBSTEP(SMC, SMI, st, CH, S0)                                          \
    CM_FRAGS(SMC, CH)                                                             \
    CM_MFMA4(hh, ah, bh) CM_COPIES(SMI, st, S0)                                   \
    CM_MFMA4(mid, ah, bl) CM_COPIES(SMI, st, S0 + 1)                              \
    CM_MFMA4(ll, al, bl) CM_COPIES(SMI, st, S0 + 2)                               \
    CM_MFMA4(mid, al, bh) CM_COPIES(SMI, st, S0 + 3)
#define CM_STEP(kt, SMC, SMI)                                                     \
    {                                                                             \
        const uint32_t st_ = (kt) + NST - 1;                                      \
        const bool cp_ = st_ < nk;                                                \
        CM_SUBSTEP(SMC, SMI, st_, ch0, 0)                                         \
        CM_SUBSTEP(SMC, SMI, st_, ch1, 4)                                         \
        if (NST == 3 && cp_) __builtin_amdgcn_s_waitcnt(0x0070 | NC);             \
        else __builtin_amdgcn_s_waitcnt(0x0070);                                  \
        __builtin_amdgcn_s_barrier();                                             \
    }
#define CM_ISSUE(SM, step)                                                        \
    _Pragma("unroll") for (int q_ = 0; q_ < NC; q_++) CM_COPY(SM, step, q_)

    uint32_t kt = 0;
    if constexpr (NST == 3) {
        CM_ISSUE(sm0, 0)
        if (nk > 1) {
            CM_ISSUE(sm1, 1)
            finish_terms();
            __builtin_amdgcn_s_waitcnt(0x0070 | NC);
        } else {
            finish_terms();
            __builtin_amdgcn_s_waitcnt(0x0070);
        }
        __builtin_amdgcn_s_barrier();
        for (; kt + 3 <= nk; kt += 3) {
            CM_STEP(kt, sm0, sm2)
            CM_STEP(kt + 1, sm1, sm0)
            CM_STEP(kt + 2, sm2, sm1)
        }
        if (kt < nk) CM_STEP(kt, sm0, sm2)
        if (kt + 1 < nk) CM_STEP(kt + 1, sm1, sm0)
    } else {
        CM_ISSUE(sm0, 0)
        finish_terms();
        __builtin_amdgcn_s_waitcnt(0x0070);
        __builtin_amdgcn_s_barrier();
        for (; kt + 2 <= nk; kt += 2) {
            CM_STEP(kt, sm0, sm1)
            CM_STEP(kt + 1, sm1, sm0)
        }
        if (kt < nk) CM_STEP(kt, sm0, sm1)
    }
    __builtin_amdgcn_s_waitcnt(0x0070);      // no copy may land after the workgroup ends
#undef CM_ISSUE
#undef CM_STEP
#undef CM_SUBSTEP
#undef CM_MFMA4
#undef CM_FRAGS
#undef CM_COPIES
#undef CM_COPY

    // ---- epilogue: one uniform dispatch to the store routine of this mode
    const uint32_t row0 = tr * TM, col0 = tc * BN;
    if (mode == kSplitFix) {
        // the slices' partials meet in the last slice to arrive; the others are done
        const uint64_t tile_id = (uint64_t)bt * ntiles + g;
        if (!split_fixup<TM>(hh, mid, ll, pout + tile_id * gridDim.z * (TM * BN), gridDim.z, kz, wave, lane,
                             tcnt + tile_id, &ticket))
            return;
        mode = kWrap;
    }
#define CM_STORE(M, P) store_wave_tile<M, P>(hh, mid, ll, rterm, cterm, bt, row0, col0, wr, wc, l32, lh, epi)
    const TileBase tb = epi.tile_base(bt, row0, col0, TM, BN);
    if (tb.base != nullptr) {           // a whole tile: the lean store
        if (mode == kWrap) store_wave_fast<kWrap>(hh, mid, ll, rterm, cterm, tb.base, tb.ld, wr, wc, l32, lh, epi.lo, epi.hi);
        else if (mode == kSatNarrow)
            store_wave_fast<kSatNarrow>(hh, mid, ll, rterm, cterm, tb.base, tb.ld, wr, wc, l32, lh, epi.lo, epi.hi);
        else store_wave_fast<kSatWide>(hh, mid, ll, rterm, cterm, tb.base, tb.ld, wr, wc, l32, lh, epi.lo, epi.hi);
    } else if (mode == kSatNarrow) {
        if (epi.pairs) CM_STORE(kSatNarrow, true); else CM_STORE(kSatNarrow, false);
    } else if (mode == kWrap) {
        if (epi.pairs) CM_STORE(kWrap, true); else CM_STORE(kWrap, false);
    } else {
        if (epi.pairs) CM_STORE(kSatWide, true); else CM_STORE(kSatWide, false);
    }
#undef CM_STORE
}

// ---------------------------------------------------------------- standard conv, few taps
// A standard convolution whose taps per output (in_ch kh kw <= 80) are few -- a network's stem
// over its 1 .. 4 input channels, the 1x1 convolutions of up to 80 channels -- straight on the
// VALU instead of im2col + GEMM (which would pad each kernel position to 16 channels, and
// whose folded 1x1 operand costs a transposing split; such products are bound by their output
// bytes, not by the multiplies): a lane per output pixel over OG output channels, its
// taps gathered once (zero outside the input) and packed in pairs, each channel's sum by
// v_dot2_i32_i16 against the channel's pairs staged in LDS (read by every lane at one
// address).  The sum is int32 where that is exact -- the wrap path (the int32 wrap is its
// rule), or a channel whose bound sum |w| 2^15 + |bias| 2^8 stays below 2^31 -- and int64
// otherwise; then floor(acc / 2^8) clamped to [lo, hi] (saturation and a fused RELU / RELU6),
// as the GEMM path stores it.  w in the packed layout of cm_conv (ConvKernel.h:136-159).
constexpr uint32_t kCsMaxTaps = 80;          // taps a lane holds (40 pairs)
// taps x output channels up to which the VALU path beats the GEMM's (measured on MobileNetV2's
// 1x1 shapes: 32 x 192 at 28^2 pixels 18 vs 21 us, 64 x 384 at 14^2 21 vs 17 us)
constexpr uint64_t kCsMaxWork = 12288;
constexpr uint32_t kCsOg = 32;               // output channels a workgroup holds at most (4 at a time)

struct ConvSmall {
    const int16_t* x;
    const int16_t* w;
    const int16_t* bias;
    int16_t* y;
    uint32_t in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, sh, sw, dh, dw, pt, pl;
    uint32_t per_m, tiles, last;             // the packed weights: entries per output channel, 16-channel
                                             // tiles, lanes of a position in the last tile
    uint32_t cs, cn, gs, wrap;
    int32_t lo, hi;
    uint32_t og;                             // output channels of a workgroup (a multiple of 4, <= kCsOg)
};

// PW: a pointwise convolution (1x1, stride 1, no padding, the output plane the input's): the
// lane's taps are its pixel in each input channel, loaded before the weights are staged.
template <uint32_t NP, bool PW>                // tap pairs, a multiple of 4 (16-byte LDS reads)
__global__ __launch_bounds__(256) void conv_small_kernel(ConvSmall c) {
    __shared__ __attribute__((aligned(16))) uint32_t wl[kCsOg][NP];
    __shared__ int32_t bl[kCsOg];
    __shared__ uint32_t exact[kCsOg], exact4[kCsOg / 4];
    __shared__ uint64_t ybase[kCsOg];         // a channel's offset in the output (the y pattern)
    const uint32_t t = threadIdx.x, plane = c.out_h * c.out_w, taps = c.in_ch * c.kh * c.kw, khw = c.kh * c.kw;
    const uint32_t oc0 = blockIdx.y * c.og, nb = blockIdx.z;
    const uint32_t og = min(c.og, c.out_ch - oc0);
    const int16_t* xb = c.x + (uint64_t)nb * c.in_ch * c.in_h * c.in_w;
    // the lane's output pixel and its taps, loaded before the weights are staged (their
    // latency under the staging's): PW from the input planes at the pixel; otherwise the taps
    // in order (ci, a, b) from running counters, the same for every lane (scalar registers),
    // so that all the loads go out at once
    const uint32_t p = blockIdx.x * 256 + t;
    const bool live = p < plane;
    uint32_t xv[NP];
    if constexpr (PW) {
#pragma unroll
        for (uint32_t pr = 0; pr < NP; pr++) {
            const uint32_t lo = live && 2 * pr < taps ? (uint32_t)(uint16_t)xb[(uint64_t)(2 * pr) * plane + p] : 0u;
            const uint32_t hi = live && 2 * pr + 1 < taps ? (uint32_t)(uint16_t)xb[(uint64_t)(2 * pr + 1) * plane + p] : 0u;
            xv[pr] = lo | (hi << 16);
        }
    } else {
        const uint32_t pc = live ? p : 0u;
        const uint32_t oh = pc / c.out_w, ow = pc - oh * c.out_w;
        const int ih0 = (int)(oh * c.sh) - (int)c.pt, iw0 = (int)(ow * c.sw) - (int)c.pl;
        // the kernel rows and columns whose input row / column lies inside the plane, as bit
        // masks (kh, kw <= 32), so that a tap's test is two shifts and an AND
        uint32_t rm = 0, cmk = 0;
        for (uint32_t a = 0; a < c.kh; a++) {
            const int ih = ih0 + (int)(a * c.dh);
            rm |= (ih >= 0 && ih < (int)c.in_h ? 1u : 0u) << a;
        }
        for (uint32_t b = 0; b < c.kw; b++) {
            const int iw = iw0 + (int)(b * c.dw);
            cmk |= (iw >= 0 && iw < (int)c.in_w ? 1u : 0u) << b;
        }
        if (!live) rm = 0;
        // the lane's offset from the window origin at row -pt, column -pl (never negative), and
        // the tap's offset from that origin, the same for every lane (scalar
        // registers, stepped as the counters run), so that a tap's load address is one add
        const uint32_t vo = oh * c.sh * c.in_w + ow * c.sw;
        int64_t uo = -((int64_t)c.pt * c.in_w + c.pl);
        const int64_t step_a = (int64_t)c.dh * c.in_w - (int64_t)c.kw * c.dw;
        const int64_t step_c = (int64_t)c.in_h * c.in_w - (int64_t)c.kh * c.dh * c.in_w;
        // the valid columns of the current kernel row, zero past the last input channel (the
        // taps past in_ch kh kw), updated only where a kernel row ends
        uint32_t ta = 0, tb = 0, ci = 0;
        uint32_t crow = (rm & 1u) ? cmk : 0u;
#pragma unroll
        for (uint32_t pr = 0; pr < NP; pr++) {
            uint32_t v2 = 0;
#pragma unroll
            for (uint32_t h = 0; h < 2; h++) {
                const bool in = (crow & (1u << tb)) != 0u;
                v2 |= (in ? (uint32_t)(uint16_t)xb[uo + (int64_t)vo] : 0u) << (16 * h);
                uo += c.dw;
                if (++tb == c.kw) {
                    tb = 0;
                    uo += step_a;
                    if (++ta == c.kh) {
                        ta = 0;
                        uo += step_c;
                        ci++;
                    }
                    crow = ci < c.in_ch && ((rm >> ta) & 1u) ? cmk : 0u;
                }
            }
            xv[pr] = v2;
        }
    }
    // the group's weights as int16 pairs in tap order (ci, a, b), zero past the taps
    for (uint32_t i = t; i < c.og * NP; i += 256) {
        const uint32_t o = i / NP, pr = i - o * NP;
        uint32_t v = 0;
#pragma unroll
        for (uint32_t h = 0; h < 2; h++) {
            const uint32_t tp = 2 * pr + h;
            if (o < og && tp < taps) {
                const uint32_t ci = tp / khw, pos = tp - ci * khw, ict = ci >> 4;
                const uint32_t lanes = ict + 1 == c.tiles ? c.last : 16u;
                v |= (uint32_t)(uint16_t)c.w[(uint64_t)(oc0 + o) * c.per_m + ict * khw * 16 + pos * lanes + (ci & 15)]
                     << (16 * h);
            }
        }
        wl[o][pr] = v;
    }
    if (t < kCsOg) bl[t] = t < og && c.bias ? (int32_t)c.bias[oc0 + t] : 0;
    __syncthreads();
    if (t < kCsOg) {
        // int32 is exact when sum |w| 2^15 + |bias| 2^8 < 2^31 (and always for the wrap rule)
        uint64_t bound = (uint64_t)(bl[t] < 0 ? -bl[t] : bl[t]) << 8;
        for (uint32_t pr = 0; pr < NP; pr++) {
            const int32_t w0 = (int16_t)(wl[t][pr] & 0xFFFF), w1 = (int16_t)(wl[t][pr] >> 16);
            bound += (uint64_t)((w0 < 0 ? -w0 : w0) + (w1 < 0 ? -w1 : w1)) << 15;
        }
        exact[t] = c.wrap || bound < ((uint64_t)1 << 31);
        const uint32_t oc = oc0 + t;
        ybase[t] = c.cn ? (uint64_t)(oc % c.cn) * c.cs + (uint64_t)(oc / c.cn) * c.gs : (uint64_t)oc * c.cs;
    }
    __syncthreads();
    if (t < kCsOg / 4) exact4[t] = exact[4 * t] & exact[4 * t + 1] & exact[4 * t + 2] & exact[4 * t + 3];
    __syncthreads();
    typedef short v2s __attribute__((ext_vector_type(2)));
    if (!live) return;                                    // no barrier follows
    int16_t* yb = c.y + (uint64_t)nb * c.out_ch * plane + p;
    // four channels at a time: four independent sums (channels past og have zero weights,
    // their stores are skipped)
    for (uint32_t o = 0; o < og; o += 4) {
        int64_t q[4];
        if (exact4[o / 4]) {
            int32_t acc[4];
#pragma unroll
            for (uint32_t j = 0; j < 4; j++) acc[j] = (int32_t)((uint32_t)bl[o + j] << 8);
#pragma unroll
            for (uint32_t pr = 0; pr < NP; pr += 4) {
#pragma unroll
                for (uint32_t j = 0; j < 4; j++) {
                    const uint4 wq = *reinterpret_cast<const uint4*>(&wl[o + j][pr]);
                    acc[j] = __builtin_amdgcn_sdot2(__builtin_bit_cast(v2s, xv[pr]), __builtin_bit_cast(v2s, wq.x), acc[j], false);
                    acc[j] = __builtin_amdgcn_sdot2(__builtin_bit_cast(v2s, xv[pr + 1]), __builtin_bit_cast(v2s, wq.y), acc[j], false);
                    acc[j] = __builtin_amdgcn_sdot2(__builtin_bit_cast(v2s, xv[pr + 2]), __builtin_bit_cast(v2s, wq.z), acc[j], false);
                    acc[j] = __builtin_amdgcn_sdot2(__builtin_bit_cast(v2s, xv[pr + 3]), __builtin_bit_cast(v2s, wq.w), acc[j], false);
                }
            }
#pragma unroll
            for (uint32_t j = 0; j < 4; j++) q[j] = acc[j] >> 8;
        } else {
#pragma unroll
            for (uint32_t j = 0; j < 4; j++) {
                long long acc = (long long)bl[o + j] * 256;
#pragma unroll
                for (uint32_t pr = 0; pr < NP; pr++) {
                    const uint32_t wv = wl[o + j][pr];
                    acc += (long long)(int16_t)(xv[pr] & 0xFFFF) * (int16_t)(wv & 0xFFFF) +
                           (long long)(int16_t)(xv[pr] >> 16) * (int16_t)(wv >> 16);
                }
                q[j] = acc >> 8;
            }
        }
#pragma unroll
        for (uint32_t j = 0; j < 4; j++)
            if (o + j < og) yb[ybase[o + j]] = (int16_t)(q[j] > c.hi ? c.hi : (q[j] < c.lo ? c.lo : q[j]));
    }
}

// ---------------------------------------------------------------- depthwise conv
__global__ __launch_bounds__(256) void conv_dw_kernel(const int16_t* __restrict__ x,
                                                      const int16_t* __restrict__ w,
                                                      const int16_t* __restrict__ bias,
                                                      int16_t* __restrict__ y, uint64_t total,
                                                      uint32_t ch, uint32_t in_h, uint32_t in_w,
                                                      uint32_t out_h, uint32_t out_w, uint32_t kh,
                                                      uint32_t kw, uint32_t sh, uint32_t sw,
                                                      uint32_t dh, uint32_t dw, uint32_t pt,
                                                      uint32_t pl, uint32_t dws, uint32_t cs,
                                                      uint32_t cn, uint32_t gs, uint32_t wrap, int32_t lo,
                                                      int32_t hi) {
    for (uint64_t o = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; o < total;
         o += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t ow = (uint32_t)(o % out_w);
        const uint64_t t1 = o / out_w;
        const uint32_t oh = (uint32_t)(t1 % out_h);
        const uint64_t t2 = t1 / out_h;
        const uint32_t c = (uint32_t)(t2 % ch);
        const uint64_t nb = t2 / ch;
        const int16_t* xp = x + (nb * ch + c) * in_h * in_w;
        const int16_t* wp = w + (uint64_t)c * dws;
        long long acc = bias ? (long long)bias[c] * 256 : 0;
        for (uint32_t a = 0; a < kh; a++) {
            const int ih = (int)(oh * sh + a * dh) - (int)pt;
            if (ih < 0 || ih >= (int)in_h) continue;
            for (uint32_t b = 0; b < kw; b++) {
                const int iw = (int)(ow * sw + b * dw) - (int)pl;
                if (iw < 0 || iw >= (int)in_w) continue;
                acc += (long long)xp[(uint64_t)ih * in_w + iw] * wp[a * kw + b];
            }
        }
        if (wrap) acc = (long long)(int32_t)(uint32_t)(unsigned long long)acc;
        long long q = acc >> 8;
        const uint64_t plane = (uint64_t)out_h * out_w;
        uint64_t base = cn ? (uint64_t)(c % cn) * cs + (uint64_t)(c / cn) * gs : (uint64_t)c * cs;
        y[nb * ch * plane + base + (uint64_t)oh * out_w + ow] = (int16_t)(q > hi ? hi : (q < lo ? lo : q));
    }
}

// Depthwise 3x3, dilation 1, stride SH x SW (the MobileNet blocks): each lane computes R
// output rows of one column (a vertical strip) from the (R - 1) SH + 3 input rows' three
// taps held in registers.  Lanes of a wavefront sit on neighbouring columns, so each load
// is one contiguous run of an input row and the L1 serves the overlap between neighbours.
// Sums are int32 where they are exact: the wrap path, or a channel whose bound
// sum |w| 2^15 + |bias| 2^8 stays below 2^31; int64 otherwise.
template <int SH, int SW, int R>
__global__ __launch_bounds__(256) void conv_dw3_kernel(const int16_t* __restrict__ x, const int16_t* __restrict__ w,
                                                       const int16_t* __restrict__ bias, int16_t* __restrict__ y,
                                                       uint32_t items, uint32_t strips, uint32_t ch, uint32_t in_h,
                                                       uint32_t in_w, uint32_t out_h, uint32_t out_w, uint32_t pt,
                                                       uint32_t pl, uint32_t dws, uint32_t cs, uint32_t cn,
                                                       uint32_t gs, uint32_t wrap, int32_t lo, int32_t hi) {
    constexpr int NR = (R - 1) * SH + 3;
    const uint32_t per_plane = strips * out_w;
    for (uint32_t it = blockIdx.x * blockDim.x + threadIdx.x; it < items; it += gridDim.x * blockDim.x) {
        const uint32_t p = it / per_plane, rem = it - p * per_plane;
        const uint32_t sidx = rem / out_w, ow = rem - sidx * out_w;
        const uint32_t nb = p / ch, c = p - nb * ch;
        const int16_t* xp = x + (uint64_t)p * in_h * in_w;
        const int16_t* wp = w + (uint64_t)c * dws;
        int wv[9];
        uint32_t wabs = 0;
#pragma unroll
        for (int i = 0; i < 9; i++) {
            wv[i] = wp[i];
            wabs += (uint32_t)(wv[i] < 0 ? -wv[i] : wv[i]);
        }
        const int b0 = bias ? (int)bias[c] : 0;
        const int oh0 = (int)(sidx * R);
        const int ih0 = oh0 * SH - (int)pt, iw0 = (int)(ow * SW) - (int)pl;
        bool cv[3];
#pragma unroll
        for (int b = 0; b < 3; b++) cv[b] = (uint32_t)(iw0 + b) < in_w;
        int v[NR][3];
#pragma unroll
        for (int r = 0; r < NR; r++) {
            const int ih = ih0 + r;
            const bool rv = (uint32_t)ih < in_h;
            const int16_t* xr = xp + (int64_t)ih * in_w + iw0;
#pragma unroll
            for (int b = 0; b < 3; b++) v[r][b] = (rv && cv[b]) ? (int)xr[b] : 0;
        }
        const uint64_t bound = (uint64_t)wabs * 32768u + (uint64_t)(b0 < 0 ? -b0 : b0) * 256u;
        int out[R];
        if (wrap || bound < ((uint64_t)1 << 31)) {
#pragma unroll
            for (int i = 0; i < R; i++) {
                uint32_t acc = (uint32_t)b0 << 8;
#pragma unroll
                for (int a = 0; a < 3; a++)
#pragma unroll
                    for (int b = 0; b < 3; b++) acc += (uint32_t)(v[i * SH + a][b] * wv[a * 3 + b]);
                out[i] = clamp_i32((int)acc >> 8, lo, hi);
            }
        } else {
#pragma unroll
            for (int i = 0; i < R; i++) {
                long long acc = (long long)b0 * 256;
#pragma unroll
                for (int a = 0; a < 3; a++)
#pragma unroll
                    for (int b = 0; b < 3; b++) acc += (long long)v[i * SH + a][b] * wv[a * 3 + b];
                const long long q = acc >> 8;
                out[i] = (int)(q > hi ? hi : (q < lo ? lo : q));
            }
        }
        const uint64_t plane = (uint64_t)out_h * out_w;
        const uint64_t base = cn ? (uint64_t)(c % cn) * cs + (uint64_t)(c / cn) * gs : (uint64_t)c * cs;
        int16_t* yp = y + (uint64_t)nb * ch * plane + base + ow;
#pragma unroll
        for (int i = 0; i < R; i++)
            if ((uint32_t)(oh0 + i) < out_h) yp[(uint64_t)(oh0 + i) * out_w] = (int16_t)out[i];
    }
}

// Depthwise 3x3 stride 1 on rows of a multiple of 8 columns: a lane computes 8 columns x R
// rows.  Per input row it loads the 16-byte word of its 8 columns and the dwords either side
// (columns 8j - 2 .. 8j + 9, zero past the row), and every output takes its row's three
// taps as two v_dot2_i32_i16 against packed weight pairs, so no 16-bit value is unpacked.
// PL (the left pad, 0..2) fixes which pairs line up.  Exact int32 sums as in
// conv_dw3_kernel; a channel whose bound leaves int32 takes int64 per value.
typedef short cm_s16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ int dot2(uint32_t x, uint32_t w, int acc) {
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(cm_s16x2, x), __builtin_bit_cast(cm_s16x2, w), acc, false);
}

__device__ __forceinline__ uint32_t pack16(int lo, int hi) { return (uint32_t)(uint16_t)lo | ((uint32_t)hi << 16); }

template <int PL, int R>
__global__ __launch_bounds__(256) void conv_dw3v_kernel(const int16_t* __restrict__ x, const int16_t* __restrict__ w,
                                                        const int16_t* __restrict__ bias, int16_t* __restrict__ y,
                                                        uint32_t items, uint32_t strips, uint32_t groups, uint32_t ch,
                                                        uint32_t in_h, uint32_t in_w, uint32_t out_h, uint32_t out_w,
                                                        uint32_t pt, uint32_t dws, uint32_t cs, uint32_t cn,
                                                        uint32_t gs, uint32_t wrap, int32_t lo, int32_t hi) {
    const uint32_t per_plane = strips * groups;
    for (uint32_t it = blockIdx.x * blockDim.x + threadIdx.x; it < items; it += gridDim.x * blockDim.x) {
        const uint32_t p = it / per_plane, rem = it - p * per_plane;
        const uint32_t sidx = rem / groups, j = rem - sidx * groups;
        const uint32_t nb = p / ch, c = p - nb * ch;
        const int16_t* xp = x + (uint64_t)p * in_h * in_w;
        const int16_t* wp = w + (uint64_t)c * dws;
        int wv[9];
        uint32_t wabs = 0;
#pragma unroll
        for (int i = 0; i < 9; i++) {
            wv[i] = wp[i];
            wabs += (uint32_t)(wv[i] < 0 ? -wv[i] : wv[i]);
        }
        const int b0 = bias ? (int)bias[c] : 0;
        const uint64_t bound = (uint64_t)wabs * 32768u + (uint64_t)(b0 < 0 ? -b0 : b0) * 256u;
        const bool exact32 = wrap || bound < ((uint64_t)1 << 31);
        const int oh0 = (int)(sidx * R);
        const uint32_t c0 = 8 * j;                                   // first output column
        const uint64_t plane = (uint64_t)out_h * out_w;
        const uint64_t base = cn ? (uint64_t)(c % cn) * cs + (uint64_t)(c / cn) * gs : (uint64_t)c * cs;
        int16_t* yp = y + (uint64_t)nb * ch * plane + base + c0;
        if (!exact32) {
            // int64 per value (weights too large for an int32 bound): each tap loaded alone
            for (int i = 0; i < R && (uint32_t)(oh0 + i) < out_h; i++) {
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    long long a64 = (long long)b0 * 256;
                    for (int a = 0; a < 3; a++) {
                        const int ih = oh0 + i - (int)pt + a;
                        if ((uint32_t)ih >= in_h) continue;
                        for (int b = 0; b < 3; b++) {
                            const int iw = (int)c0 + t - PL + b;
                            if ((uint32_t)iw < in_w) a64 += (long long)xp[(uint64_t)ih * in_w + iw] * wv[3 * a + b];
                        }
                    }
                    const long long v = a64 >> 8;
                    yp[(uint64_t)(oh0 + i) * out_w + t] = (int16_t)(v > hi ? hi : (v < lo ? lo : v));
                }
            }
            continue;
        }
        // weight pairs per kernel row: (w0, w1), (w2, 0) for an even first tap; (0, w0), (w1, w2) odd
        uint32_t wA[3], wB[3], wC[3], wD[3];
#pragma unroll
        for (int a = 0; a < 3; a++) {
            wA[a] = pack16(wv[3 * a], wv[3 * a + 1]);
            wB[a] = pack16(wv[3 * a + 2], 0);
            wC[a] = pack16(0, wv[3 * a]);
            wD[a] = pack16(wv[3 * a + 1], wv[3 * a + 2]);
        }
        int acc[R][8];
#pragma unroll
        for (int i = 0; i < R; i++)
#pragma unroll
            for (int t = 0; t < 8; t++) acc[i][t] = b0 * 256;
#pragma unroll
        for (int r = 0; r < R + 2; r++) {
            const int ih = oh0 - (int)pt + r;
            uint32_t W[6] = {0, 0, 0, 0, 0, 0};                      // columns c0 - 2 .. c0 + 9
            if ((uint32_t)ih < in_h) {
                const int16_t* xr = xp + (uint64_t)ih * in_w + c0;
                if (c0 + 8 <= in_w) {
                    const int4 mid = *reinterpret_cast<const int4*>(xr);
                    W[1] = (uint32_t)mid.x;
                    W[2] = (uint32_t)mid.y;
                    W[3] = (uint32_t)mid.z;
                    W[4] = (uint32_t)mid.w;
                }
                if (c0 >= 2) W[0] = *reinterpret_cast<const uint32_t*>(xr - 2);
                if (c0 + 10 <= in_w) W[5] = *reinterpret_cast<const uint32_t*>(xr + 8);
            }
#pragma unroll
            for (int a = 0; a < 3; a++) {
                const int i = r - a;                                   // the output row fed at tap row a
                if (i < 0 || i >= R) continue;
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    const int q0 = t - PL + 2;                         // window index of tap b = 0
                    if ((q0 & 1) == 0) {
                        acc[i][t] = dot2(W[q0 >> 1], wA[a], acc[i][t]);
                        acc[i][t] = dot2(W[(q0 >> 1) + 1], wB[a], acc[i][t]);
                    } else {
                        acc[i][t] = dot2(W[q0 >> 1], wC[a], acc[i][t]);
                        acc[i][t] = dot2(W[(q0 >> 1) + 1], wD[a], acc[i][t]);
                    }
                }
            }
        }
#pragma unroll
        for (int i = 0; i < R; i++) {
            if ((uint32_t)(oh0 + i) >= out_h) break;
            int q[8];
#pragma unroll
            for (int t = 0; t < 8; t++) q[t] = clamp_i32(acc[i][t] >> 8, lo, hi);
            int4 o;
            o.x = __builtin_bit_cast(int, __builtin_amdgcn_cvt_pk_i16(q[0], q[1]));
            o.y = __builtin_bit_cast(int, __builtin_amdgcn_cvt_pk_i16(q[2], q[3]));
            o.z = __builtin_bit_cast(int, __builtin_amdgcn_cvt_pk_i16(q[4], q[5]));
            o.w = __builtin_bit_cast(int, __builtin_amdgcn_cvt_pk_i16(q[6], q[7]));
            store_stream(yp + (uint64_t)(oh0 + i) * out_w, o);
        }
    }
}

// ---------------------------------------------------------------- skinny products (int32 wrap)
// C = sat16(wrap32(A . B) >> 8) for A of at most 32 rows: the decode step's linears, where a
// 128-column MFMA tile would be mostly padding and the plane split would cost more than the
// product.  The wrap rule makes the int32 sum mod 2^32 exact in any order, so v_dot2_i32_i16
// (two products per lane-op, no clamp) accumulates it directly and split k needs no care.
// A wavefront takes 128 columns (a pair per lane) and one slice of kSkinnyKc k; A's rows of
// the slice sit in LDS as k pairs, read as broadcasts.  B layouts (BL): 0 row-major [k][m]
// and 1 the packed 32-column tiles (one 4-byte load per k row for the lane's two columns,
// paired by byte permutes); 2 transposed [m][k] (a column's k contiguous: 16-byte loads of
// 8 k).  Every B load of the slice is issued before the first product.  With several slices
// each wavefront writes its int32 partials [slice][ks][n][m] for skinny_reduce_kernel.
constexpr uint32_t kSkinnyKc = 64;
constexpr uint32_t kSkinnySegs = 4;

// The products of one skinny launch: up to kSkinnySegs B / C / m over the same A rows (batch 1),
// or one product over `batch` slices.  Segment s owns column blocks [cb0[s], cb0[s + 1]) of
// the grid and output pairs [pair0[s], pair0[s + 1]) of the reduce.
struct SkinnySegs {
    const int16_t* b[kSkinnySegs];
    int16_t* c[kSkinnySegs];
    int32_t* part[kSkinnySegs];
    uint32_t m[kSkinnySegs], cb0[kSkinnySegs];
    uint64_t pair0[kSkinnySegs];
    uint32_t count;
};

template <int NR, int BL>
__global__ __launch_bounds__(64) void skinny_wrap_kernel(const int16_t* __restrict__ a, uint64_t a_bs,
                                                          SkinnySegs segs, uint64_t b_bs, uint64_t c_bs, uint32_t n,
                                                          uint32_t k) {
    constexpr uint32_t KP = kSkinnyKc / 2;                                // k pairs per slice
    __shared__ __attribute__((aligned(16))) uint32_t sa[NR][KP];
    uint32_t si = 0;                                                      // this workgroup's segment
    for (uint32_t i = 1; i < segs.count; i++)
        if (blockIdx.x >= segs.cb0[i]) si = i;
    const int16_t* __restrict__ b = segs.b[si];
    int16_t* __restrict__ c = segs.c[si];
    int32_t* __restrict__ part = segs.part[si];
    const uint32_t m = segs.m[si];
    const uint32_t lane = threadIdx.x, cb = blockIdx.x - segs.cb0[si], ks = blockIdx.y, bt = blockIdx.z,
                   nks = gridDim.y;
    const uint32_t k0 = ks * kSkinnyKc, k1 = min(k, k0 + kSkinnyKc);
    const int16_t* ab = a + bt * a_bs;
    const int16_t* bb = b + bt * b_bs;
    const uint32_t j0 = cb * 128 + 2 * lane;
    const bool live = j0 < m;
    // B's pairs (B[kk][j], B[kk+1][j]) of the slice for columns j0 and j0 + 1
    uint32_t p0[KP], p1[KP];
    if (BL == 2) {
#pragma unroll
        for (uint32_t q = 0; q < KP / 4; q++) {
            const uint32_t kk = k0 + 8 * q;
            int4 x = make_int4(0, 0, 0, 0), y = make_int4(0, 0, 0, 0);
            if (live && kk < k1) {                          // k1 - k0 is a multiple of 8 here
                x = *reinterpret_cast<const int4*>(bb + (uint64_t)j0 * k + kk);
                y = *reinterpret_cast<const int4*>(bb + (uint64_t)(j0 + 1) * k + kk);
            }
            p0[4 * q] = x.x; p0[4 * q + 1] = x.y; p0[4 * q + 2] = x.z; p0[4 * q + 3] = x.w;
            p1[4 * q] = y.x; p1[4 * q + 1] = y.y; p1[4 * q + 2] = y.z; p1[4 * q + 3] = y.w;
        }
    } else {
#pragma unroll
        for (uint32_t i = 0; i < KP; i++) {
            const uint32_t kk = k0 + 2 * i;
            uint32_t w0 = 0, w1 = 0;
            if (live && kk < k1) {                          // k1 - k0 is even
                const uint64_t o0 = BL == 1 ? ((uint64_t)(j0 >> 5) * k + kk) * 32 + (j0 & 31) : (uint64_t)kk * m + j0;
                const uint64_t o1 = BL == 1 ? o0 + 32 : o0 + m;
                w0 = *reinterpret_cast<const uint32_t*>(bb + o0);
                w1 = *reinterpret_cast<const uint32_t*>(bb + o1);
            }
            p0[i] = __builtin_amdgcn_perm(w1, w0, 0x05040100u);
            p1[i] = __builtin_amdgcn_perm(w1, w0, 0x07060302u);
        }
    }
    // A's rows of the slice (zero past n and past k)
    for (uint32_t e = lane; e < NR * KP; e += 64) {
        const uint32_t r = e / KP, kk = k0 + 2 * (e - r * KP);
        sa[r][e - r * KP] = (r < n && kk < k1) ? *reinterpret_cast<const uint32_t*>(ab + (uint64_t)r * k + kk) : 0u;
    }
    __syncthreads();
    typedef short v2s __attribute__((ext_vector_type(2)));
    int acc0[NR], acc1[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) acc0[r] = acc1[r] = 0;
#pragma unroll
    for (uint32_t i = 0; i < KP; i += 4) {
#pragma unroll
        for (int r = 0; r < NR; r++) {
            const uint4 av = *reinterpret_cast<const uint4*>(&sa[r][i]);
            const uint32_t a4[4] = {av.x, av.y, av.z, av.w};
#pragma unroll
            for (int t = 0; t < 4; t++) {
                acc0[r] = __builtin_amdgcn_sdot2(__builtin_bit_cast(v2s, a4[t]), __builtin_bit_cast(v2s, p0[i + t]),
                                                 acc0[r], false);
                acc1[r] = __builtin_amdgcn_sdot2(__builtin_bit_cast(v2s, a4[t]), __builtin_bit_cast(v2s, p1[i + t]),
                                                 acc1[r], false);
            }
        }
    }
    int16_t* cbt = c + bt * c_bs;
    auto store = [&](uint32_t r, int s0, int s1) {
        const int q0 = min(max(s0 >> 8, -32768), 32767), q1 = min(max(s1 >> 8, -32768), 32767);
        *reinterpret_cast<uint32_t*>(cbt + (uint64_t)r * m + j0) = (uint32_t)(uint16_t)q0 | ((uint32_t)q1 << 16);
    };
    if (nks == 1) {
        if (live) {
#pragma unroll
            for (int r = 0; r < NR; r++)
                if ((uint32_t)r < n) store(r, acc0[r], acc1[r]);
        }
        return;
    }
    if (!live) return;
    const uint64_t per = (uint64_t)n * m;
    int32_t* pp = part + ((uint64_t)bt * nks + ks) * per;
#pragma unroll
    for (int r = 0; r < NR; r++)
        if ((uint32_t)r < n) *reinterpret_cast<int2*>(pp + (uint64_t)r * m + j0) = make_int2(acc0[r], acc1[r]);
}

// Sums the int32 partials of the k slices (wrapping) and applies the output rule: a lane per
// pair of outputs.
__global__ __launch_bounds__(256) void skinny_reduce_kernel(SkinnySegs segs, uint64_t c_bs, uint32_t n,
                                                            uint32_t nks, uint32_t batch, uint64_t total) {
    for (uint64_t e = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (uint64_t)gridDim.x * blockDim.x) {
        uint32_t si = 0;
        for (uint32_t j = 1; j < segs.count; j++)
            if (e >= segs.pair0[j]) si = j;
        const uint64_t per = (uint64_t)n * segs.m[si], pairs = per / 2, el = e - segs.pair0[si];
        const uint64_t bt = el / pairs, i = 2 * (el - bt * pairs);
        int16_t* c = segs.c[si];
        const int32_t* pp = segs.part[si] + bt * nks * per + i;
        uint32_t s0 = 0, s1 = 0;
        uint32_t q = 0;
        for (; q + 8 <= nks; q += 8) {                 // eight slices' loads in flight at once
            int2 v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = *reinterpret_cast<const int2*>(pp + (uint64_t)(q + u) * per);
#pragma unroll
            for (int u = 0; u < 8; u++) {
                s0 += (uint32_t)v[u].x;
                s1 += (uint32_t)v[u].y;
            }
        }
        for (; q < nks; q++) {
            const int2 v = *reinterpret_cast<const int2*>(pp + (uint64_t)q * per);
            s0 += (uint32_t)v.x;
            s1 += (uint32_t)v.y;
        }
        const int q0 = min(max((int)s0 >> 8, -32768), 32767), q1 = min(max((int)s1 >> 8, -32768), 32767);
        *reinterpret_cast<uint32_t*>(c + bt * c_bs + i) = (uint32_t)(uint16_t)q0 | ((uint32_t)q1 << 16);
    }
}

// ---------------------------------------------------------------- skinny products on split weights
// C = sat16(wrap32(A . B) >> 8) for A of at most 16 rows against a weight already split into
// byte planes (cm_matmul_split_b).  Sixteen rows are exactly one v_mfma_i32_16x16x64_i8
// operand, so the products run on MFMA over limbs with the plane GEMM's recombination, and a
// workgroup owns NB 16-column blocks for the whole k: its W wavefronts take the 64-k steps w,
// w + W, .. (the loads of a chunk of sp_chunk(NB) steps all in flight before the chunk's products)
// and add their wrapped partials in LDS, so there are no partial buffers and no second launch.
// A is split in registers, 16 k of row l % 16 per lane (the MFMA operand layout), its row sums
// taken on the way; B's column sums come from the plane image.  Everything the stores of a
// thread's first kSpPre output elements read besides the product (B's column sums, the output
// job's parameter entry and x) is loaded before the products, under the weight loads.  NB
// trades the workgroups a weight's columns give (one MFMA block each: narrow weights) against
// the A rows every workgroup reads again (wide ones).
// 64-k steps whose loads a wavefront issues together, wavefronts of an NB-block workgroup (the
// register budget of its launch bounds), and the output elements a thread prefetches for
__host__ __device__ constexpr uint32_t sp_chunk(uint32_t nb) { return nb == 4 ? 2u : 4u; }
__host__ __device__ constexpr uint32_t sp_max_waves(uint32_t nb) { return nb == 1 ? 16u : 8u; }
__host__ __device__ constexpr uint32_t sp_pre(uint32_t nb) { return nb == 1 ? 1u : 2u; }

struct SkinnyPlaneSegs {
    const int8_t* hi[kSkinnySegs];
    const int8_t* lo[kSkinnySegs];
    const int32_t* part[kSkinnySegs];
    int16_t* c[kSkinnySegs];
    uint32_t m[kSkinnySegs], lines_p[kSkinnySegs], cb0[kSkinnySegs];
    uint32_t count;
};

// A row-ops COPY / ADDX job applied to a one-product launch's output as it is stored: out[r][j]
// = copy_addx(x[r][j], C[r][j]) with the job's op word (A kind, output kind, flags), its
// parameter block and bq_sh (the residual add of a decode linear); out == nullptr: none.
struct SkinnyAddx {
    const uint8_t* x;
    uint8_t* out;
    const uint8_t* params;
    uint32_t op, bq_sh;
};

// The operands of one output element's store other than the product, as loaded (nothing
// waits for them before the weight loads go out): B's column sums of the first kSpSlabs slabs,
// the output job's parameter entry and x (int16 or int32).
constexpr uint32_t kSpSlabs = 4;
struct SkinnyEpiIn {
    uint32_t cs[kSpSlabs] = {0, 0, 0, 0};
    uint4 prm{};
    int32_t x = 0;
};

// The wrapped partial products of one skinny workgroup: NB 16-column blocks whose plane lines
// start at bh[b] / bl[b] (the block's first column), into red [W][16][16 NB] and A's row sums
// into rsum [W][16]; ends with the workgroup barrier.  SAT: each wavefront's three limb sums
// (exact in int32) into red [3][W][16][16 NB] -- HH, MID, LL -- for the exact recombination.
template <uint32_t NB, bool SAT = false>
__device__ __forceinline__ void skinny_products(const int16_t* __restrict__ a, uint32_t n, uint32_t k, uint32_t kp,
                                                const int8_t* const (&bh)[NB], const int8_t* const (&bl)[NB],
                                                uint32_t* red, int32_t* rsum) {
    constexpr uint32_t COLS = 16 * NB, CH = sp_chunk(NB);
    const uint32_t W = blockDim.x >> 6, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t r = lane & 15, g = lane >> 4;             // A row and B column of a block; k group
    const uint32_t nsteps = kp / 64;
    const bool row_ok = r < n;
    const int16_t* arow = a + (uint64_t)(row_ok ? r : 0) * k;
    const int4 pad8 = make_int4(0x00800080, 0x00800080, 0x00800080, 0x00800080);   // eight kPad: A' = 0
    v4i hh[NB], mid[NB], ll[NB];
#pragma unroll
    for (uint32_t b = 0; b < NB; b++) hh[b] = mid[b] = ll[b] = v4i{0, 0, 0, 0};
    int32_t asum = 0;
    for (uint32_t s0 = wave; s0 < nsteps; s0 += W * CH) {
        int4 av[CH][2];
        v4i bhv[CH][NB], blv[CH][NB];
#pragma unroll
        for (uint32_t u = 0; u < CH; u++) {
            const uint32_t st = s0 + u * W;
            const bool live = st < nsteps;
            const uint32_t kk = (live ? st : 0) * 64 + 16 * g;
            // k % 8 == 0: each half of the lane's 16 k is wholly real or wholly past k; a half past
            // k loads row 0's first 8 (in bounds) and takes the pad instead
            const bool h0 = live && row_ok && kk + 8 <= k, h1 = live && row_ok && kk + 16 <= k;
            const int4 a0 = *reinterpret_cast<const int4*>(arow + (h0 ? kk : 0));
            const int4 a1 = *reinterpret_cast<const int4*>(arow + (h1 ? kk + 8 : 0));
            av[u][0] = h0 ? a0 : pad8;
            av[u][1] = h1 ? a1 : pad8;
#pragma unroll
            for (uint32_t b = 0; b < NB; b++) {
                const uint64_t off = (uint64_t)r * kp + kk;
                bhv[u][b] = *reinterpret_cast<const v4i*>(bh[b] + off);
                blv[u][b] = *reinterpret_cast<const v4i*>(bl[b] + off);
            }
        }
#pragma unroll
        for (uint32_t u = 0; u < CH; u++) {
            if (s0 + u * W >= nsteps) break;                  // wave-uniform
            const uint32_t kk = (s0 + u * W) * 64 + 16 * g;
            if (row_ok && kk + 8 <= k) asum += sum8(av[u][0]);
            if (row_ok && kk + 16 <= k) asum += sum8(av[u][1]);
            uint2 h0, l0, h1, l1;
            split8(av[u][0], h0, l0);
            split8(av[u][1], h1, l1);
            const v4i ah{(int)h0.x, (int)h0.y, (int)h1.x, (int)h1.y}, al{(int)l0.x, (int)l0.y, (int)l1.x, (int)l1.y};
#pragma unroll
            for (uint32_t b = 0; b < NB; b++) hh[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah, bhv[u][b], hh[b], 0, 0, 0);
#pragma unroll
            for (uint32_t b = 0; b < NB; b++) mid[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah, blv[u][b], mid[b], 0, 0, 0);
#pragma unroll
            for (uint32_t b = 0; b < NB; b++) ll[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(al, blv[u][b], ll[b], 0, 0, 0);
#pragma unroll
            for (uint32_t b = 0; b < NB; b++) mid[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(al, bhv[u][b], mid[b], 0, 0, 0);
        }
    }
    // this wavefront's wrapped partials: lane l holds column l % 16 of each block, rows 4 g .. + 3
#pragma unroll
    for (uint32_t b = 0; b < NB; b++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t e = (wave * 16 + 4 * g + i) * COLS + 16 * b + r;
            if constexpr (SAT) {
                const uint32_t plane = W * 16 * COLS;
                red[e] = (uint32_t)hh[b][i];
                red[plane + e] = (uint32_t)mid[b][i];
                red[2 * plane + e] = (uint32_t)ll[b][i];
            } else {
                red[e] = ((uint32_t)hh[b][i] << 16) + ((uint32_t)mid[b][i] << 8) + (uint32_t)ll[b][i];
            }
        }
    asum += __shfl_xor(asum, 16, 64);
    asum += __shfl_xor(asum, 32, 64);
    if (g == 0) rsum[wave * 16 + r] = asum;
    __syncthreads();
}

// C[row][col] of a skinny workgroup from its wavefronts' partials (column cl of the tile), A's
// row sums and B's column sum cs.
__device__ __forceinline__ int16_t skinny_value(const uint32_t* red, const int32_t* rsum, uint32_t W, uint32_t cols,
                                                uint32_t row, uint32_t cl, uint32_t k, uint32_t cs) {
    uint32_t acc = 0u - 16384u * k, rs = 0;
    for (uint32_t w = 0; w < W; w++) {
        acc += red[(w * 16 + row) * cols + cl];
        rs += (uint32_t)rsum[w * 16 + row];
    }
    acc += 128u * rs + 128u * cs;
    return (int16_t)min(max((int32_t)acc >> 8, -32768), 32767);
}

// The same by the saturating rule: the wavefronts' limb sums (red [3][W][16][cols]) and the
// row / column sums recombined exactly in int64 (each term is exact in int32: |A|, |B| <=
// 2^15 and k <= 32768), then floor(acc / 2^8) saturated to int16.
__device__ __forceinline__ int16_t skinny_value_sat(const uint32_t* red, const int32_t* rsum, uint32_t W,
                                                    uint32_t cols, uint32_t row, uint32_t cl, uint32_t k,
                                                    uint32_t cs) {
    const uint32_t plane = W * 16 * cols;
    long long acc = -16384ll * k, rs = 0;
    for (uint32_t w = 0; w < W; w++) {
        const uint32_t e = (w * 16 + row) * cols + cl;
        acc += ((long long)(int32_t)red[e] << 16) + ((long long)(int32_t)red[plane + e] << 8) +
               (long long)(int32_t)red[2 * plane + e];
        rs += rsum[w * 16 + row];
    }
    acc += 128ll * rs + 128ll * (int32_t)cs;
    const long long q = acc >> 8;
    return (int16_t)(q > 32767 ? 32767 : (q < -32768 ? -32768 : q));
}

// B's column sum of column col from the slabs a prefetch took (the first kSpSlabs) and the rest.
__device__ __forceinline__ uint32_t skinny_colsum(const uint32_t (&pre)[kSpSlabs], const int32_t* part, uint32_t nslab,
                                                  uint32_t lp, uint32_t col) {
    uint32_t cs = 0;
#pragma unroll
    for (uint32_t sl = 0; sl < kSpSlabs; sl++) cs += pre[sl];
    for (uint32_t sl = kSpSlabs; sl < nslab; sl++) cs += (uint32_t)part[(uint64_t)sl * lp + col];
    return cs;
}

// XK: the output job's x kind (0: no job, 1: int16, 2: int32); SAT: the saturating rule (no job).
template <uint32_t NB, uint32_t XK, bool SAT = false>
__global__ __launch_bounds__(64 * sp_max_waves(NB)) void skinny_planes_kernel(const int16_t* __restrict__ a, uint32_t n,
                                                                       uint32_t k, uint32_t kp, uint32_t nslab,
                                                                       SkinnyPlaneSegs segs, SkinnyAddx ax) {
    constexpr uint32_t COLS = 16 * NB;
    extern __shared__ __attribute__((aligned(16))) uint32_t sp_lds[];
    const uint32_t W = blockDim.x >> 6;
    static_assert(!SAT || XK == 0, "no output job on the saturating products");
    uint32_t* red = sp_lds;                                  // [W][16][COLS] wrapped partials ([3][..] SAT)
    int32_t* rsum = reinterpret_cast<int32_t*>(sp_lds + (SAT ? 3 : 1) * W * 16 * COLS);   // [W][16] A row sums
    uint32_t si = 0;
    for (uint32_t i = 1; i < segs.count; i++)
        if (blockIdx.x >= segs.cb0[i]) si = i;
    const uint32_t c0 = (blockIdx.x - segs.cb0[si]) * COLS;
    const uint32_t m = segs.m[si], lp = segs.lines_p[si];
    const int32_t* __restrict__ part = segs.part[si];
    const uint32_t ck = (ax.op >> 8) & 3;
    const bool pb = (ax.op & ro::F_P_BCAST) != 0;
    // element e of the tile: row e / COLS, column c0 + e % COLS
    auto epi_in = [&](uint32_t e) {
        SkinnyEpiIn in;
        const uint32_t row = e / COLS, col = c0 + e % COLS;
        if (row >= n || col >= m) return in;
#pragma unroll
        for (uint32_t sl = 0; sl < kSpSlabs; sl++)
            if (sl < nslab) in.cs[sl] = (uint32_t)part[(uint64_t)sl * lp + col];
        if constexpr (XK != 0) {
            in.prm = *reinterpret_cast<const uint4*>(ax.params + 16u * (pb ? 0u : col));
            const uint64_t ex = (uint64_t)row * m + col;
            if constexpr (XK == 1) in.x = reinterpret_cast<const int16_t*>(ax.x)[ex];
            else in.x = reinterpret_cast<const int32_t*>(ax.x)[ex];
        }
        return in;
    };
    constexpr uint32_t PRE = sp_pre(NB);
    SkinnyEpiIn pre[PRE];
#pragma unroll
    for (uint32_t i = 0; i < PRE; i++) pre[i] = epi_in(threadIdx.x + i * blockDim.x);
    const int8_t* bh[NB];
    const int8_t* bl[NB];
#pragma unroll
    for (uint32_t b = 0; b < NB; b++) {
        bh[b] = segs.hi[si] + (uint64_t)(c0 + 16 * b) * kp;
        bl[b] = segs.lo[si] + (uint64_t)(c0 + 16 * b) * kp;
    }
    skinny_products<NB, SAT>(a, n, k, kp, bh, bl, red, rsum);
    int16_t* __restrict__ c = segs.c[si];
    auto store = [&](uint32_t e, const SkinnyEpiIn& in) {
        const uint32_t row = e / COLS, cl = e - row * COLS, col = c0 + cl;
        if (row >= n || col >= m) return;
        const uint32_t cs = skinny_colsum(in.cs, part, nslab, lp, col);
        const int16_t y = SAT ? skinny_value_sat(red, rsum, W, COLS, row, cl, k, cs)
                              : skinny_value(red, rsum, W, COLS, row, cl, k, cs);
        const uint64_t eo = (uint64_t)row * m + col;
        c[eo] = y;
        if constexpr (XK != 0) {
            const ro::i64 o = ro::copy_addx(in.x, y, ro::param_of(in.prm), ax.op, ax.bq_sh, ck);
            if (ck == 0) reinterpret_cast<int16_t*>(ax.out)[eo] = (int16_t)o;
            else reinterpret_cast<int32_t*>(ax.out)[eo] = (int32_t)o;
        }
    };
#pragma unroll
    for (uint32_t i = 0; i < PRE; i++)
        if (threadIdx.x + i * blockDim.x < 16 * COLS) store(threadIdx.x + i * blockDim.x, pre[i]);
    for (uint32_t e = threadIdx.x + PRE * blockDim.x; e < 16 * COLS; e += blockDim.x) store(e, epi_in(e));
}

// The MULACT job over a gate and an up product of the same A (segments 0 and 1, m columns
// each): a workgroup's NB blocks are NB / 2 blocks of gate columns and the same columns of up,
// and its stores write both products and out = MULACT(gate, up) with the job's parameters.
struct SkinnyMulact {
    int16_t* out;
    const uint8_t* params;
    uint32_t bcast;
    const uint8_t* tab;       // the row-ops table image (the sigmoid)
};

struct SkinnyPairIn {
    uint32_t cg[kSpSlabs] = {0, 0, 0, 0}, cu[kSpSlabs] = {0, 0, 0, 0};
    uint4 prm{};
};

template <uint32_t NB>
__global__ __launch_bounds__(64 * sp_max_waves(NB)) void skinny_mulact_kernel(const int16_t* __restrict__ a, uint32_t n,
                                                                        uint32_t k, uint32_t kp, uint32_t nslab,
                                                                        SkinnyPlaneSegs segs, SkinnyMulact mj) {
    constexpr uint32_t COLS = 16 * NB, H = COLS / 2;
    extern __shared__ __attribute__((aligned(16))) uint32_t sp_lds[];
    const uint32_t W = blockDim.x >> 6;
    uint32_t* red = sp_lds;
    int32_t* rsum = reinterpret_cast<int32_t*>(sp_lds + W * 16 * COLS);
    const uint32_t c0 = blockIdx.x * H, m = segs.m[0], lp = segs.lines_p[0];
    auto epi_in = [&](uint32_t e) {
        SkinnyPairIn in;
        const uint32_t row = e / H, col = c0 + e % H;
        if (row >= n || col >= m) return in;
#pragma unroll
        for (uint32_t sl = 0; sl < kSpSlabs; sl++)
            if (sl < nslab) {
                in.cg[sl] = (uint32_t)segs.part[0][(uint64_t)sl * lp + col];
                in.cu[sl] = (uint32_t)segs.part[1][(uint64_t)sl * segs.lines_p[1] + col];
            }
        in.prm = *reinterpret_cast<const uint4*>(mj.params + 16u * (mj.bcast ? 0u : col));
        return in;
    };
    const SkinnyPairIn pre = epi_in(threadIdx.x);
    const int8_t* bh[NB];
    const int8_t* bl[NB];
#pragma unroll
    for (uint32_t b = 0; b < NB; b++) {
        const uint32_t sg = b < NB / 2 ? 0u : 1u, cb = c0 + 16 * (b % (NB / 2));
        bh[b] = segs.hi[sg] + (uint64_t)cb * kp;
        bl[b] = segs.lo[sg] + (uint64_t)cb * kp;
    }
    skinny_products<NB>(a, n, k, kp, bh, bl, red, rsum);
    auto store = [&](uint32_t e, const SkinnyPairIn& in) {
        const uint32_t row = e / H, cl = e - row * H, col = c0 + cl;
        if (row >= n || col >= m) return;
        const int16_t gv = skinny_value(red, rsum, W, COLS, row, cl, k, skinny_colsum(in.cg, segs.part[0], nslab, lp, col));
        const int16_t uv = skinny_value(red, rsum, W, COLS, row, H + cl, k,
                                        skinny_colsum(in.cu, segs.part[1], nslab, segs.lines_p[1], col));
        const uint64_t eo = (uint64_t)row * m + col;
        segs.c[0][eo] = gv;
        segs.c[1][eo] = uv;
        mj.out[eo] = (int16_t)ro::mulact_elem(gv, uv, ro::param_of(in.prm), mj.tab);
    };
    if (threadIdx.x < 16 * H) store(threadIdx.x, pre);
    for (uint32_t e = threadIdx.x + blockDim.x; e < 16 * H; e += blockDim.x) store(e, epi_in(e));
}

// ---------------------------------------------------------------- drivers
// Byte planes [slices][lines_p][kp] of one operand and its partial line sums
// [slices][nslab][lines_p].
struct Planes {
    int8_t *hi, *lo;
    int32_t* part;
    uint32_t lines_p, kp, nslab, slices;
    uint32_t tile = 128;                 // GEMM tile rows when this is the A operand
    uint32_t rows = 0;                   // real lines (the rest up to lines_p are padding)
    uint32_t sums = 0;                   // partial line sums per line (0: one per slab)
    uint32_t nsum() const { return sums ? sums : nslab; }
    size_t bytes() const {
        return (size_t)slices * lines_p * kp * 2 + (size_t)slices * nslab * lines_p * 4 + 1024;
    }
    void carve(char*& p) {
        hi = reinterpret_cast<int8_t*>(p); p += (size_t)slices * lines_p * kp;
        lo = reinterpret_cast<int8_t*>(p); p += (size_t)slices * lines_p * kp;
        part = reinterpret_cast<int32_t*>(p); p += (size_t)slices * nslab * lines_p * 4;
        p = reinterpret_cast<char*>(round_up(reinterpret_cast<uintptr_t>(p), 256));
    }
};

template <class Src, bool KFast>
int run_split(const Src& src, uint64_t src_slice, Planes& pl, hipStream_t s) {
    CM_LAUNCH("split_kernel", (split_kernel<Src, KFast>), dim3(pl.lines_p / 64, pl.nslab, pl.slices), dim3(256),
                       0, s, src, src_slice, pl.hi, pl.lo, pl.part, pl.lines_p, pl.kp, pl.nslab);
    return CM_OK;
}

// Tile rows of the GEMM for an n x m output of `batch` slices.  A 256-row tile (8 waves, one
// workgroup per compute unit) has the most operand reuse, but a grid of them that does not
// fill the compute units in whole rounds leaves most of the last round idle; 128-row tiles
// (two workgroups per unit) then finish sooner.  Outputs of at most 64 rows take 64-row tiles.
uint32_t gemm_tile_rows(uint32_t n, uint32_t m, uint32_t batch, uint32_t cus) {
    if (n <= 64) return 64;
    if (n <= 128) return 128;
    const uint64_t tiles = (uint64_t)ceil_div(n, 256) * ceil_div(m, BN) * batch;
    return (tiles % cus == 0 || tiles >= 4ull * cus) ? 256 : 128;
}

template <class Epi>
int run_gemm(const Planes& A, const Planes& B, uint32_t batch, uint32_t k, Epi epi, hipStream_t s,
             int32_t* pout = nullptr, uint32_t ksteps = 0, uint32_t* tcnt = nullptr) {
    const uint32_t tm = A.tile;
    const uint32_t tiles_r = ceil_div(A.rows, tm), tiles_c = B.lines_p / BN;
    if (tm != 64 && tm != 128 && tm != 256) return fail(CM_EINVAL, "gemm: tile rows %u", tm);
    if ((uint64_t)tiles_r * tm > A.lines_p) return fail(CM_EINVAL, "gemm: %u tile rows past %u plane rows", tm, A.lines_p);
    const uint64_t a_slice = A.slices > 1 ? (uint64_t)A.lines_p * A.kp : 0;
    const uint64_t b_slice = B.slices > 1 ? (uint64_t)B.lines_p * B.kp : 0;
    const uint64_t rp_slice = A.slices > 1 ? (uint64_t)A.nslab * A.lines_p : 0;
    const uint64_t cp_slice = B.slices > 1 ? (uint64_t)B.nslab * B.lines_p : 0;
    if (ksteps && tcnt == nullptr) return fail(CM_EINVAL, "gemm: a split over k needs the arrival counts");
    const uint32_t mode = ksteps ? kSplitFix : (epi.wrap ? kWrap : (k <= 8192 ? kSatNarrow : kSatWide));
    const uint32_t nz = ksteps ? ceil_div(A.kp / BK, ksteps) : 1;
    const dim3 grid(tiles_r * tiles_c, batch, nz);
    if (tm == 256) {
        CM_LAUNCH("gemm_planes_kernel", (gemm_planes_kernel<4, 3, Epi>), grid, dim3(512), 0, s, A.hi, A.lo, A.part,
                  a_slice, rp_slice, A.lines_p, B.hi, B.lo, B.part, b_slice, cp_slice, B.lines_p, B.nslab, A.nsum(),
                  tiles_r, tiles_c, A.kp, (int32_t)(64 * k), mode, pout, ksteps, tcnt, epi);
    } else if (tm == 64) {
        CM_LAUNCH("gemm_planes_kernel", (gemm_planes_kernel<1, 2, Epi>), grid, dim3(128), 0, s, A.hi, A.lo, A.part,
                  a_slice, rp_slice, A.lines_p, B.hi, B.lo, B.part, b_slice, cp_slice, B.lines_p, B.nslab, A.nsum(),
                  tiles_r, tiles_c, A.kp, (int32_t)(64 * k), mode, pout, ksteps, tcnt, epi);
    } else {
        CM_LAUNCH("gemm_planes_kernel", (gemm_planes_kernel<2, 2, Epi>), grid, dim3(256), 0, s, A.hi, A.lo, A.part,
                  a_slice, rp_slice, A.lines_p, B.hi, B.lo, B.part, b_slice, cp_slice, B.lines_p, B.nslab, A.nsum(),
                  tiles_r, tiles_c, A.kp, (int32_t)(64 * k), mode, pout, ksteps, tcnt, epi);
    }
    return CM_OK;
}

// k steps per slice for a wrap-mode matmul whose output tiles leave most workgroup slots
// idle (0: no split): slices until the grid about fills the slots, at least 4 steps each.
uint32_t gemm_ksteps(uint32_t tm, uint32_t tiles, uint32_t kp, const DeviceState* st) {
    const uint32_t slots = st->cus * (tm == 256 ? 1u : 2u), nk = kp / BK;
    if (tiles * 2 > slots || nk < 16) return 0;
    const uint32_t nz = std::min(slots / tiles, nk / 4);
    if (nz < 2) return 0;
    return ceil_div(nk, nz);
}

Planes make_planes(uint32_t lines, uint32_t kp, uint32_t slices, uint32_t align = 128) {
    Planes p{};
    p.lines_p = (uint32_t)round_up(lines, align);
    p.rows = lines;
    p.kp = kp;
    p.nslab = ceil_div(kp, SLAB);
    p.slices = slices;
    p.tile = align;
    return p;
}

}  // namespace
}  // namespace cm

namespace cm {
namespace {

int matmul_check(uint32_t k, uint32_t gemv_kw, int64_t a_bs, int64_t b_bs, int64_t c_bs, uint32_t b_packed = 0) {
    // the limb sums HL + LH stay exact in int32 for k <= 32768
    if (k == 0 || k > 32768) return fail(CM_EINVAL, "matmul: k = %u outside 1 .. 32768", k);
    if (gemv_kw && gemv_kw != 1 && gemv_kw != 2 && gemv_kw != 4 && gemv_kw != 8)
        return fail(CM_EINVAL, "matmul: gemv_kw %u", gemv_kw);
    if (gemv_kw > 1 && (k % (16 * gemv_kw)))
        return fail(CM_EINVAL, "matmul: k %u not a multiple of 16 * gemv_kw", k);
    if (b_packed > 2 || (b_packed && gemv_kw)) return fail(CM_EINVAL, "matmul: b_packed %u with gemv_kw %u", b_packed, gemv_kw);
    if (a_bs < 0 || b_bs < 0 || c_bs < 0) return fail(CM_EINVAL, "matmul: negative batch stride");
    return CM_OK;
}

// Planes of rows with k contiguous (lda elements apart, 16-byte aligned): the short-row
// kernel for kp <= 256, else a wavefront per row and slab.
int split_row_lines(const int16_t* a, Slices a_slice, uint64_t lda, uint32_t n, uint32_t k, Planes& P,
                    hipStream_t s) {
    if (P.kp <= 256) {
#define CM_SHORT(G)                                                                                            \
    CM_LAUNCH("split_rows_kernel", split_rows_short_kernel<G>, dim3(ceil_div(P.lines_p, 4 * (64 / G)), 1, P.slices), \
              dim3(256), 0, s, a, a_slice, lda, n, k, P.hi, P.lo, P.part, P.lines_p, P.kp)
        if (P.kp == 64) { CM_SHORT(8); } else if (P.kp == 128) { CM_SHORT(16); } else { CM_SHORT(32); }
#undef CM_SHORT
        return CM_OK;
    }
    CM_LAUNCH("split_rows_kernel", split_rows_kernel, dim3(P.lines_p / 4, P.nslab, P.slices), dim3(256), 0, s, a,
              a_slice, lda, n, k, P.hi, P.lo, P.part, P.lines_p, P.kp, P.nslab);
    return CM_OK;
}

// A's planes: row-major [n][k] slices at a_slice elements (0: one slice).
int split_a(const int16_t* a, uint64_t a_slice, uint32_t n, uint32_t k, Planes& A, hipStream_t s) {
    if (aligned16(a) && (k & 7) == 0 && (a_slice & 7) == 0) return split_row_lines(a, Slices{a_slice}, k, n, k, A, s);
    return run_split<SrcRowMajor, true>(SrcRowMajor{a, n, k, k}, a_slice, A, s);
}

// B's planes from its image (row-major, packed 32-column tiles or the GEMV image).
int split_b(const int16_t* b, uint64_t b_slice, uint32_t k, uint32_t m, uint32_t b_packed, uint32_t gemv_kw,
            Planes& B, hipStream_t s) {
    const uint32_t layout = gemv_kw ? 2 : (b_packed == 2 ? 3 : (b_packed ? 1 : 0));
    if (layout == 3 && aligned16(b) && (b_slice & 7) == 0 && (k & 7) == 0)
        return split_row_lines(b, Slices{b_slice}, k, m, k, B, s);    // B's lines are rows with k contiguous
    const bool fast_b = aligned16(b) && (b_slice & 7) == 0 &&
                        (layout == 1 || (layout == 0 && (m & 7) == 0) || (layout == 2 && gemv_kw == 1 && (m & 7) == 0));
    if (fast_b) {
        CM_LAUNCH("split_cols_kernel", split_cols_kernel, dim3(B.lines_p / 32, B.nslab, B.slices), dim3(256), 0, s,
                  b, Slices{b_slice}, (uint64_t)m, layout == 1 ? 1u : 0u, m, k, B.hi, B.lo, B.part, B.lines_p, B.kp,
                  B.nslab);
        return CM_OK;
    }
    return run_split<SrcMatB, false>(SrcMatB{b, m, k, m, layout, gemv_kw}, b_slice, B, s);
}

// The skinny path of cm_matmul (wrap32, n <= 32): slices of kSkinnyKc k.
// Skinny products of the same A (n rows, k) into `count` segments, or one product over
// `batch` slices (count 1); the partials of all segments in one workspace, one reduce launch.
int skinny_run(const int16_t* a, uint32_t n, uint32_t k, uint32_t batch, int64_t a_bs, int64_t b_bs, int64_t c_bs,
               uint32_t count, const int16_t* const* b, int16_t* const* c, const uint32_t* m, uint32_t b_packed,
               DeviceState* st, hipStream_t s, const WsRegion* fixed = nullptr) {
    const uint32_t nks = ceil_div(k, kSkinnyKc);
    SkinnySegs segs{};
    segs.count = count;
    uint32_t cbs = 0;
    uint64_t pairs = 0;
    size_t pbytes = 0;
    for (uint32_t i = 0; i < count; i++) {
        segs.b[i] = b[i];
        segs.c[i] = c[i];
        segs.m[i] = m[i];
        segs.cb0[i] = cbs;
        segs.pair0[i] = pairs;
        cbs += ceil_div(m[i], 128);
        pairs += (uint64_t)batch * n * m[i] / 2;
        pbytes += (size_t)batch * nks * n * m[i] * 4;
    }
    if (nks > 65535 || batch > 65535) return fail(CM_EINVAL, "matmul: skinny grid %u x %u x %u", cbs, nks, batch);
    if (nks > 1) {
        void* ws;
        int rc = take_workspace(st, fixed, pbytes, &ws, s);
        if (rc) return rc;
        int32_t* p = static_cast<int32_t*>(ws);
        for (uint32_t i = 0; i < count; i++) {
            segs.part[i] = p;
            p += (size_t)batch * nks * n * m[i];
        }
    }
    const dim3 grid(cbs, nks, batch);
#define CM_SKINNY(NR, BL)                                                                                         \
    CM_LAUNCH("skinny_wrap_kernel", (skinny_wrap_kernel<NR, BL>), grid, dim3(64), 0, s, a, (uint64_t)a_bs, segs,   \
              (uint64_t)b_bs, (uint64_t)c_bs, n, k)
#define CM_SKINNY_BL(NR) \
    if (b_packed == 2) { CM_SKINNY(NR, 2); } else if (b_packed) { CM_SKINNY(NR, 1); } else { CM_SKINNY(NR, 0); }
    if (n <= 8) { CM_SKINNY_BL(8) } else if (n <= 16) { CM_SKINNY_BL(16) } else { CM_SKINNY_BL(32) }
#undef CM_SKINNY_BL
#undef CM_SKINNY
    if (nks > 1) {
        const unsigned blocks = (unsigned)std::min<uint64_t>((pairs + 255) / 256, (uint64_t)st->cus * 8);
        CM_LAUNCH("skinny_reduce_kernel", skinny_reduce_kernel, dim3(blocks), dim3(256), 0, s, segs, (uint64_t)c_bs,
                  n, nks, batch, pairs);
    }
    return CM_OK;
}

int skinny_wrap(const int16_t* a, const int16_t* b, int16_t* c, uint32_t n, uint32_t k, uint32_t m, uint32_t batch,
                int64_t a_bs, int64_t b_bs, int64_t c_bs, uint32_t b_packed, DeviceState* st, hipStream_t s,
                const WsRegion* fixed) {
    return skinny_run(a, n, k, batch, a_bs, b_bs, c_bs, 1, &b, &c, &m, b_packed, st, s, fixed);
}

// The wrap-mode split over k for a matmul of this shape: k steps per slice (0: none) and the
// bytes of its int32 partials.
uint32_t matmul_ksteps(const Planes& A, const Planes& B, uint32_t n, uint32_t m, uint32_t batch, uint32_t wrap32,
                       const DeviceState* st, size_t* bytes) {
    const uint32_t tiles = ceil_div(n, A.tile) * (B.lines_p / BN) * batch;
    const uint32_t ks = wrap32 ? gemm_ksteps(A.tile, tiles, A.kp, st) : 0;
    // the partials of every slice, whole tiles (split_fixup's layout)
    *bytes = ks ? (size_t)ceil_div(A.kp / BK, ks) * tiles * A.tile * BN * 4 : 0;
    return ks;
}

int gemm_out(const Planes& A, const Planes& B, int16_t* c, uint32_t n, uint32_t k, uint32_t m, uint32_t batch,
             int64_t c_bs, uint32_t wrap32, hipStream_t s, const DeviceState* st, int32_t* pout = nullptr,
             uint32_t ksteps = 0) {
    const bool pairs = (reinterpret_cast<uintptr_t>(c) & 3) == 0 && (m & 1) == 0 && (c_bs & 1) == 0;
    EpiMatmul epi{c, (uint64_t)c_bs, n, m, wrap32 ? 1u : 0u, pairs ? 1u : 0u};
    // a split product is finished by the last slice of each tile (one launch): an arrival
    // count per tile (a split has at most one tile per compute unit, gemm_ksteps)
    const uint64_t tiles = (uint64_t)ceil_div(A.rows, A.tile) * (B.lines_p / BN) * batch;
    if (ksteps && tiles > st->split_cnt_n)
        return fail(CM_EINVAL, "gemm: %llu split tiles past the %u arrival counts", (unsigned long long)tiles,
                    st->split_cnt_n);
    return run_gemm(A, B, batch, k, epi, s, pout, ksteps, ksteps ? st->split_cnt : nullptr);
}

}  // namespace
}  // namespace cm

namespace cm {
namespace {

// cm_matmul with its workspace from `fixed` (nullptr: the grow-only workspace).
int matmul_run(const int16_t* a, const int16_t* b, int16_t* c, uint32_t n, uint32_t k, uint32_t m, uint32_t batch,
               int64_t a_bs, int64_t b_bs, int64_t c_bs, uint32_t b_packed, uint32_t gemv_kw, uint32_t wrap32,
               hipStream_t s, DeviceState* st, const WsRegion* fixed) {
    if (n == 0 || m == 0 || batch == 0) return CM_OK;
    int rc = matmul_check(k, gemv_kw, a_bs, b_bs, c_bs, b_packed);
    if (rc) return rc;
    if (wrap32 && n <= 32 && gemv_kw == 0 && (m & 1) == 0 && (k & 1) == 0 && (reinterpret_cast<uintptr_t>(a) & 3) == 0 &&
        (reinterpret_cast<uintptr_t>(b) & 3) == 0 && (reinterpret_cast<uintptr_t>(c) & 3) == 0 && (a_bs & 1) == 0 &&
        (b_bs & 1) == 0 && (c_bs & 1) == 0 && (b_packed != 1 || (m & 31) == 0) &&
        (b_packed != 2 || ((k & 7) == 0 && aligned16(b) && (b_bs & 7) == 0)))
        return skinny_wrap(a, b, c, n, k, m, batch, a_bs, b_bs, c_bs, b_packed, st, s, fixed);
    const uint32_t kp = (uint32_t)round_up(k, BK);
    const uint32_t sa = (batch > 1 && a_bs != 0) ? batch : 1, sb = (batch > 1 && b_bs != 0) ? batch : 1;
    Planes A = make_planes(n, kp, sa, gemm_tile_rows(n, m, batch, st->cus)), B = make_planes(m, kp, sb);
    size_t pbytes;
    const uint32_t ksteps = matmul_ksteps(A, B, n, m, batch, wrap32, st, &pbytes);
    void* ws;
    rc = take_workspace(st, fixed, A.bytes() + B.bytes() + pbytes, &ws, s);
    if (rc) return rc;
    char* p = static_cast<char*>(ws);
    A.carve(p);
    B.carve(p);
    const uint64_t a_slice = sa > 1 ? (uint64_t)a_bs : 0, b_slice = sb > 1 ? (uint64_t)b_bs : 0;
    rc = split_a(a, a_slice, n, k, A, s);
    if (rc) return rc;
    rc = split_b(b, b_slice, k, m, b_packed, gemv_kw, B, s);
    if (rc) return rc;
    return gemm_out(A, B, c, n, k, m, batch, c_bs, wrap32, s, st, reinterpret_cast<int32_t*>(p), ksteps);
}

// The no-allocation scratch: every call of cm_matmul_noalloc on a device takes its planes, line
// sums and split-k partials from that device's copy of this array (the code object holds one
// per device from load to process end).  Host code never passes `scratch` itself: its
// device address per device comes from hipGetSymbolAddress at set-up (DeviceState::scratch).
constexpr size_t kScratchBytes = CM_NOALLOC_MAX_BYTES;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

// The arrival counts of the split-k products finished in place (kSplitFix), one per output
// tile and batch slice of a launch: zero from load, and every launch leaves them zero (the
// last slice of a tile resets its count), so they need no clearing between launches or graph
// replays.  Launches that overlap on one device (other streams) must not both split.
constexpr uint32_t kSplitCounts = 16384;
static __device__ __align__(256) uint32_t split_counts[kSplitCounts];

}  // namespace

int gemm_scratch_setup(DeviceState* st) {
    void* ptr = nullptr;
    CM_HIP_CHECK(hipGetSymbolAddress((void**)&ptr, HIP_SYMBOL(scratch)));
    if (ptr == nullptr || (reinterpret_cast<uintptr_t>(ptr) & 255))
        return fail(CM_EHIP, "no-allocation scratch: unusable device address %p", ptr);
    st->scratch = ptr;
    st->scratch_bytes = kScratchBytes;
    void* cp = nullptr;
    CM_HIP_CHECK(hipGetSymbolAddress(&cp, HIP_SYMBOL(split_counts)));
    if (cp == nullptr) return fail(CM_EHIP, "split-k arrival counts: no device address");
    st->split_cnt = static_cast<uint32_t*>(cp);
    st->split_cnt_n = kSplitCounts;
    return CM_OK;
}

}  // namespace cm

extern "C" int cm_matmul(const int16_t* a, const int16_t* b, int16_t* c, uint32_t n, uint32_t k,
                         uint32_t m, uint32_t batch, int64_t a_bs, int64_t b_bs, int64_t c_bs,
                         uint32_t b_packed, uint32_t gemv_kw, uint32_t wrap32, void* stream) {
    using namespace cm;
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    return matmul_run(a, b, c, n, k, m, batch, a_bs, b_bs, c_bs, b_packed, gemv_kw, wrap32, as_stream(stream), st,
                      nullptr);
}

extern "C" int cm_matmul_noalloc(const int16_t* a, const int16_t* b, int16_t* c, uint32_t n, uint32_t k,
                                 uint32_t m, uint32_t batch, int64_t a_bs, int64_t b_bs, int64_t c_bs,
                                 uint32_t b_packed, uint32_t gemv_kw, uint32_t wrap32, void* stream) {
    using namespace cm;
    DeviceState* st;
    int rc = state_ready(&st);                       // no set-up here: that allocates the unit tables
    if (rc) return rc;
    if (st->scratch == nullptr) return fail(CM_EINVAL, "no-allocation scratch not set up on this device");
    const WsRegion region{st->scratch, st->scratch_bytes};
    return matmul_run(a, b, c, n, k, m, batch, a_bs, b_bs, c_bs, b_packed, gemv_kw, wrap32, as_stream(stream), st,
                      &region);
}

extern "C" size_t cm_matmul_b_planes_bytes(uint32_t k, uint32_t m, uint32_t b_slices) {
    using namespace cm;
    if (k == 0 || m == 0 || b_slices == 0) return 0;
    return make_planes(m, (uint32_t)round_up(k, BK), b_slices).bytes();
}

extern "C" int cm_matmul_split_b(const int16_t* b, void* planes, uint32_t k, uint32_t m, uint32_t b_slices,
                                 int64_t b_bs, uint32_t b_packed, uint32_t gemv_kw, void* stream) {
    using namespace cm;
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    if (m == 0 || b_slices == 0) return CM_OK;
    rc = matmul_check(k, gemv_kw, 0, b_bs, 0, b_packed);
    if (rc) return rc;
    if (reinterpret_cast<uintptr_t>(planes) & 255) return fail(CM_EALIGN, "matmul: b planes not 256-byte aligned");
    Planes B = make_planes(m, (uint32_t)round_up(k, BK), b_slices);
    char* p = static_cast<char*>(planes);
    B.carve(p);
    return split_b(b, b_slices > 1 ? (uint64_t)b_bs : 0, k, m, b_packed, gemv_kw, B, as_stream(stream));
}

extern "C" int cm_matmul_planes(const int16_t* a, const void* b_planes, int16_t* c, uint32_t n, uint32_t k,
                                uint32_t m, uint32_t batch, int64_t a_bs, uint32_t b_slices, int64_t c_bs,
                                uint32_t wrap32, void* stream) {
    using namespace cm;
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    if (n == 0 || m == 0 || batch == 0) return CM_OK;
    rc = matmul_check(k, 0, a_bs, 0, c_bs);
    if (rc) return rc;
    if (b_slices != 1 && b_slices != batch) return fail(CM_EINVAL, "matmul: %u b slices for batch %u", b_slices, batch);
    if (reinterpret_cast<uintptr_t>(b_planes) & 255) return fail(CM_EALIGN, "matmul: b planes not 256-byte aligned");
    hipStream_t s = as_stream(stream);
    const uint32_t kp = (uint32_t)round_up(k, BK);
    const uint32_t sa = (batch > 1 && a_bs != 0) ? batch : 1;
    Planes A = make_planes(n, kp, sa, gemm_tile_rows(n, m, batch, st->cus)), B = make_planes(m, kp, b_slices);
    size_t pbytes;
    const uint32_t ksteps = matmul_ksteps(A, B, n, m, batch, wrap32, st, &pbytes);
    void* ws;
    rc = workspace(st, A.bytes() + pbytes, &ws, s);
    if (rc) return rc;
    char* p = static_cast<char*>(ws);
    A.carve(p);
    char* q = static_cast<char*>(const_cast<void*>(b_planes));
    B.carve(q);
    rc = split_a(a, sa > 1 ? (uint64_t)a_bs : 0, n, k, A, s);
    if (rc) return rc;
    return gemm_out(A, B, c, n, k, m, batch, c_bs, wrap32, s, st, reinterpret_cast<int32_t*>(p), ksteps);
}

extern "C" size_t cm_matmul_a_planes_bytes(uint32_t n, uint32_t k, uint32_t nsum) {
    return cm::a_planes_bytes(n, k, nsum);
}

extern "C" int cm_matmul_aplanes(const void* a_planes, uint32_t nsum, const void* b_planes, int16_t* c, uint32_t n,
                                 uint32_t k, uint32_t m, uint32_t wrap32, void* stream) {
    using namespace cm;
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    if (n == 0 || m == 0) return CM_OK;
    rc = matmul_check(k, 0, 0, 0, 0);
    if (rc) return rc;
    if ((k % BK) || nsum == 0 || nsum > 64) return fail(CM_EINVAL, "matmul: A planes of k %u (a multiple of 64), %u sums", k, nsum);
    if ((reinterpret_cast<uintptr_t>(a_planes) & 255) || (reinterpret_cast<uintptr_t>(b_planes) & 255))
        return fail(CM_EALIGN, "matmul: planes not 256-byte aligned");
    hipStream_t s = as_stream(stream);
    const APlanes ap = a_planes_view(const_cast<void*>(a_planes), n, k, nsum);
    Planes A = make_planes(n, k, 1, gemm_tile_rows(n, m, 1, st->cus)), B = make_planes(m, k, 1);
    A.hi = ap.hi;
    A.lo = ap.lo;
    A.part = ap.part;
    A.lines_p = ap.lines;
    A.sums = nsum;
    char* q = static_cast<char*>(const_cast<void*>(b_planes));
    B.carve(q);
    size_t pbytes;
    const uint32_t ksteps = matmul_ksteps(A, B, n, m, 1, wrap32, st, &pbytes);
    void* ws = nullptr;
    if (pbytes) {
        rc = workspace(st, pbytes, &ws, s);
        if (rc) return rc;
    }
    return gemm_out(A, B, c, n, k, m, 1, 0, wrap32, s, st, static_cast<int32_t*>(ws), ksteps);
}

namespace cm {
namespace {

struct ConvGeom {
    uint32_t batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, sh, sw, dh, dw, pt, pl;
    uint32_t cs, cn, gs, wrap;          // the y pattern (cs = plane without one), int32 wrap
    uint32_t plane() const { return out_h * out_w; }
    // 1x1 stride-1 unpadded, same plane in and out, no y pattern: the images fold into the
    // GEMM's columns (one slice of batch * plane lines)
    bool fold() const {
        return kh == 1 && kw == 1 && sh == 1 && sw == 1 && pt == 0 && pl == 0 && out_h == in_h && out_w == in_w &&
               cn == 0 && cs == plane() && (uint64_t)batch * plane() < ((uint64_t)1 << 31);
    }
};

// k of the GEMM: 16-channel tiles x kernel positions (the packed weight order), in BK steps.
uint32_t conv_kp(uint32_t in_ch, uint32_t kh, uint32_t kw) {
    return (uint32_t)round_up((uint64_t)((in_ch + 15) / 16) * kh * kw * 16, BK);
}

Planes conv_b_planes(const ConvGeom& g, uint32_t kp) {
    return g.fold() ? make_planes(g.batch * g.plane(), kp, 1) : make_planes(g.plane(), kp, g.batch);
}

uint32_t conv_tile(const ConvGeom& g, const Planes& B, const DeviceState* st) {
    return gemm_tile_rows(g.out_ch, B.rows, B.slices, st->cus);
}

// The weights' planes: rows = output channels in the packed tile-major order (ConvKernel.h:136-159).
int conv_split_w(const int16_t* w, Planes& A, uint32_t out_ch, uint32_t in_ch, uint32_t kh, uint32_t kw,
                 hipStream_t s) {
    const uint32_t tiles = (in_ch + 15) / 16;
    const uint32_t rem = in_ch - (tiles - 1) * 16, last = rem <= 8 ? 8 : 16;
    const uint32_t per_m = kh * kw * ((tiles - 1) * 16 + last);
    return run_split<SrcConvW, true>(SrcConvW{w, out_ch, in_ch, kh, kw, tiles, per_m, last}, 0, A, s);
}

// The input's planes (im2col, or the folded 1x1 form) and the GEMM with the weights' planes A.
int conv_gemm(const int16_t* x, const Planes& A, Planes& B, const int16_t* bptr, int16_t* y, const ConvGeom& g,
              const DeviceState* st, hipStream_t s, int32_t lo, int32_t hi) {
    const uint32_t plane = g.plane();
    const uint64_t img = (uint64_t)g.out_ch * plane;
    if (g.fold()) {
        const uint32_t cols = g.batch * plane;
        if (B.lines_p / 64 >= 4 * st->cus) {
            // lines enough for the workgroups of whole slabs to fill the chip
            CM_LAUNCH("split_fold_kernel", split_fold_lds_kernel, dim3(B.lines_p / 64, B.nslab), dim3(256), 0, s, x,
                      g.in_ch, plane, (uint64_t)g.in_ch * plane, cols, B.hi, B.lo, B.part, B.lines_p, B.kp);
        } else if (B.lines_p / 64 >= (uint32_t)st->cus) {
            // one wave per 64 k of the slab
            const uint32_t waves = std::min<uint32_t>(16, ceil_div(std::min<uint32_t>(B.kp, SLAB), 64));
            CM_LAUNCH("split_fold_kernel", split_fold_kernel, dim3(B.lines_p / 64, B.nslab), dim3(64 * waves), 0, s,
                      x, g.in_ch, plane, (uint64_t)g.in_ch * plane, cols, B.hi, B.lo, B.part, B.lines_p, B.kp);
        } else {
            // few lines: 16 a workgroup
            const uint32_t waves = std::min<uint32_t>(16, ceil_div(std::min<uint32_t>(B.kp, SLAB), 64));
            CM_LAUNCH("split_fold_kernel", split_fold16_kernel, dim3(B.lines_p / 16, B.nslab), dim3(64 * waves), 0,
                      s, x, g.in_ch, plane, (uint64_t)g.in_ch * plane, cols, B.hi, B.lo, B.part, B.lines_p, B.kp);
        }
        const bool pairs = (reinterpret_cast<uintptr_t>(y) & 3) == 0 && (plane & 1) == 0;
        EpiConv epi{y, bptr, img, g.out_ch, cols, plane, 0, 0, g.wrap, pairs ? 1u : 0u, plane, lo, hi};
        return run_gemm(A, B, 1, g.in_ch * g.kh * g.kw, epi, s);
    }
    SrcIm2col im{x, g.in_ch, g.in_h, g.in_w, g.out_w, g.kh, g.kw, g.sh, g.sw, g.dh, g.dw, g.pt, g.pl, plane};
    int rc = run_split<SrcIm2col, false>(im, (uint64_t)g.in_ch * g.in_h * g.in_w, B, s);
    if (rc) return rc;
    const bool pairs = (reinterpret_cast<uintptr_t>(y) & 3) == 0 && (plane & 1) == 0 && (g.cs & 1) == 0 &&
                       (g.gs & 1) == 0 && (img & 1) == 0;
    EpiConv epi{y, bptr, img, g.out_ch, plane, g.cs, g.cn, g.gs, g.wrap, pairs ? 1u : 0u, 0, lo, hi};
    return run_gemm(A, B, g.batch, g.in_ch * g.kh * g.kw, epi, s);
}

// The output bounds of a fused activation (the VectorOP act codes RELU = 1, RELU6 = 2, applied
// to the raw int16 result: VectorOP ops 4 and 5 on the conv's output); CM_EINVAL otherwise.
int act_bounds(uint32_t act, int32_t& lo, int32_t& hi) {
    lo = -32768;
    hi = 32767;
    if (act == 0) return CM_OK;
    if (act == 1 || act == 2) {
        lo = 0;
        if (act == 2) hi = 6 << 8;
        return CM_OK;
    }
    return fail(CM_EINVAL, "conv: act %u (0 none, 1 RELU, 2 RELU6)", act);
}

}  // namespace
}  // namespace cm

namespace cm {
namespace {

int conv_run(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y, uint32_t batch, uint32_t in_ch,
             uint32_t in_h, uint32_t in_w, uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
             uint32_t stride_h, uint32_t stride_w, uint32_t dilation_h, uint32_t dilation_w, uint32_t pad_top,
             uint32_t pad_left, uint32_t has_bias, uint32_t is_depthwise, uint32_t y_cs, uint32_t y_cn,
             uint32_t y_gs, uint32_t wrap32, uint32_t act, void* stream) {
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    int32_t lo, hi;
    rc = act_bounds(act, lo, hi);
    if (rc) return rc;
    if (batch == 0 || out_ch == 0 || out_h == 0 || out_w == 0) return CM_OK;
    if (kh == 0 || kw == 0 || kh > 7 || kw > 7) return fail(CM_EINVAL, "conv: kernel %ux%u outside 1..7", kh, kw);
    if (stride_h == 0 || stride_w == 0 || dilation_h == 0 || dilation_w == 0)
        return fail(CM_EINVAL, "conv: zero stride or dilation");
    if ((y_cs || y_cn) && batch != 1) return fail(CM_EINVAL, "conv: y pattern needs batch 1");
    if (is_depthwise && in_ch != out_ch) return fail(CM_EINVAL, "conv: depthwise in_ch %u != out_ch %u", in_ch, out_ch);
    if (in_ch == 0) return fail(CM_EINVAL, "conv: in_ch 0");
    hipStream_t s = as_stream(stream);
    const uint32_t plane = out_h * out_w;
    const uint32_t cs = y_cs ? y_cs : plane;
    const int16_t* bptr = has_bias ? bias : nullptr;
    const bool dw3 = is_depthwise && kh == 3 && kw == 3 && dilation_h == 1 && dilation_w == 1;
    if (dw3 && stride_h == 1 && stride_w == 1 && pad_left <= 2 && (in_w & 7) == 0 && (out_w & 7) == 0 &&
        aligned16(x) && aligned16(y) && (cs & 7) == 0 && (!y_cn || (y_gs & 7) == 0)) {
        constexpr uint32_t R = 4;
        const uint32_t strips = (out_h + R - 1) / R, groups = out_w / 8;
        const uint64_t items = (uint64_t)batch * out_ch * strips * groups;
        if (items < ((uint64_t)1 << 31)) {
            const unsigned blocks = (unsigned)std::min<uint64_t>((items + 255) / 256, 65536ull * 8);
#define CM_DW3V(PL)                                                                                              \
    CM_LAUNCH("conv_dw3v_kernel", (conv_dw3v_kernel<PL, R>), dim3(blocks), dim3(256), 0, s, x, w, bptr, y,       \
              (uint32_t)items, strips, groups, out_ch, in_h, in_w, out_h, out_w, pad_top, 16u, cs, y_cn, y_gs, \
              wrap32 ? 1u : 0u, lo, hi)
            if (pad_left == 0) { CM_DW3V(0); }
            else if (pad_left == 1) { CM_DW3V(1); }
            else { CM_DW3V(2); }
#undef CM_DW3V
            return CM_OK;
        }
    }
    if (dw3 && stride_h == stride_w && stride_h <= 2) {
        const uint32_t R = stride_h == 1 ? 8 : 4;
        const uint32_t strips = (out_h + R - 1) / R;
        const uint64_t items = (uint64_t)batch * out_ch * strips * out_w;
        if (items < ((uint64_t)1 << 31)) {
            const unsigned blocks = (unsigned)std::min<uint64_t>((items + 255) / 256, 65536ull * 8);
            if (stride_h == 1) {
                CM_LAUNCH("conv_dw3_kernel", (conv_dw3_kernel<1, 1, 8>), dim3(blocks), dim3(256), 0, s, x, w, bptr, y,
                          (uint32_t)items, strips, out_ch, in_h, in_w, out_h, out_w, pad_top, pad_left, 16u, cs, y_cn,
                          y_gs, wrap32 ? 1u : 0u, lo, hi);
            } else {
                CM_LAUNCH("conv_dw3_kernel", (conv_dw3_kernel<2, 2, 4>), dim3(blocks), dim3(256), 0, s, x, w, bptr, y,
                          (uint32_t)items, strips, out_ch, in_h, in_w, out_h, out_w, pad_top, pad_left, 16u, cs, y_cn,
                          y_gs, wrap32 ? 1u : 0u, lo, hi);
            }
            return CM_OK;
        }
    }
    if (is_depthwise) {
        const uint64_t total = (uint64_t)batch * out_ch * plane;
        uint64_t blocks = (total + 255) / 256;
        if (blocks > 65536ull * 8) blocks = 65536ull * 8;
        CM_LAUNCH("conv_dw_kernel", conv_dw_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, w, bptr, y, total,
                           out_ch, in_h, in_w, out_h, out_w, kh, kw, stride_h, stride_w, dilation_h,
                           dilation_w, pad_top, pad_left, (kh * kw + 7) & ~7u, cs, y_cn, y_gs,
                           wrap32 ? 1u : 0u, lo, hi);
        return CM_OK;
    }
    if (in_ch * kh * kw <= kCsMaxTaps && (uint64_t)in_ch * kh * kw * out_ch <= kCsMaxWork && batch <= 65535 &&
        (uint64_t)in_ch * in_h * in_w < (1ull << 31) && kh <= 32 && kw <= 32 &&
        (uint64_t)out_h * stride_h * in_w + (uint64_t)out_w * stride_w < (1ull << 31)) {
        // few taps: straight on the VALU
        const uint32_t taps = in_ch * kh * kw, tiles = (in_ch + 15) / 16;
        const uint32_t rem = in_ch - (tiles - 1) * 16, last = rem <= 8 ? 8u : 16u;
        const uint32_t np = (uint32_t)round_up(ceil_div(taps, 2), 4);
        // output channels a workgroup: 32 over planes of at least 56 x 56 (the pixels' taps
        // loaded once for more channels), 16 below, 4 where 16 would leave most compute units
        // idle (a small CNN's 14 x 14 planes at batch 1)
        const uint64_t pblocks = (uint64_t)ceil_div(plane, 256) * batch;
        const uint32_t og = pblocks * ceil_div(out_ch, 16) < (uint64_t)st->cus ? 4u : (plane >= 3136 ? 32u : 16u);
        const ConvSmall cv{x, w, bptr, y, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, stride_h, stride_w,
                           dilation_h, dilation_w, pad_top, pad_left, kh * kw * ((tiles - 1) * 16 + last), tiles, last,
                           cs, y_cn, y_gs, wrap32 ? 1u : 0u, lo, hi, og};
        const dim3 grid(ceil_div(plane, 256), ceil_div(out_ch, og), batch);
        const bool pw = kh == 1 && kw == 1 && stride_h == 1 && stride_w == 1 && pad_top == 0 && pad_left == 0 &&
                        in_h == out_h && in_w == out_w;
#define CM_CS(NP_)                                                                                              \
    case NP_:                                                                                                   \
        if (pw) { CM_LAUNCH("conv_small_kernel", (conv_small_kernel<NP_, true>), grid, dim3(256), 0, s, cv); }   \
        else { CM_LAUNCH("conv_small_kernel", (conv_small_kernel<NP_, false>), grid, dim3(256), 0, s, cv); }     \
        return CM_OK;
        switch (np) {
            CM_CS(4) CM_CS(8) CM_CS(12) CM_CS(16) CM_CS(20) CM_CS(24) CM_CS(28) CM_CS(32) CM_CS(36) CM_CS(40)
        default: break;
        }
#undef CM_CS
    }
    if ((uint64_t)in_ch * kh * kw > 32768)
        return fail(CM_EINVAL, "conv: in_ch * kh * kw = %u above 32768", in_ch * kh * kw);
    const ConvGeom g{batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, stride_h, stride_w, dilation_h,
                     dilation_w, pad_top, pad_left, cs, y_cn, y_gs, wrap32 ? 1u : 0u};
    const uint32_t kp = conv_kp(in_ch, kh, kw);
    Planes B = conv_b_planes(g, kp);
    Planes A = make_planes(out_ch, kp, 1, conv_tile(g, B, st));
    void* ws;
    rc = workspace(st, A.bytes() + B.bytes(), &ws, s);
    if (rc) return rc;
    char* p = static_cast<char*>(ws);
    A.carve(p);
    B.carve(p);
    rc = conv_split_w(w, A, out_ch, in_ch, kh, kw, s);
    if (rc) return rc;
    return conv_gemm(x, A, B, bptr, y, g, st, s, lo, hi);
}

}  // namespace
}  // namespace cm

extern "C" int cm_conv(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y,
                       uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w, uint32_t out_ch,
                       uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw, uint32_t stride_h,
                       uint32_t stride_w, uint32_t dilation_h, uint32_t dilation_w, uint32_t pad_top,
                       uint32_t pad_left, uint32_t has_bias, uint32_t is_depthwise, uint32_t y_cs,
                       uint32_t y_cn, uint32_t y_gs, uint32_t wrap32, void* stream) {
    return cm::conv_run(x, w, bias, y, batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, stride_h, stride_w,
                        dilation_h, dilation_w, pad_top, pad_left, has_bias, is_depthwise, y_cs, y_cn, y_gs, wrap32,
                        0, stream);
}

extern "C" int cm_conv_act(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y, uint32_t batch,
                           uint32_t in_ch, uint32_t in_h, uint32_t in_w, uint32_t out_ch, uint32_t out_h,
                           uint32_t out_w, uint32_t kh, uint32_t kw, uint32_t stride_h, uint32_t stride_w,
                           uint32_t dilation_h, uint32_t dilation_w, uint32_t pad_top, uint32_t pad_left,
                           uint32_t has_bias, uint32_t is_depthwise, uint32_t y_cs, uint32_t y_cn, uint32_t y_gs,
                           uint32_t wrap32, uint32_t act, void* stream) {
    return cm::conv_run(x, w, bias, y, batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, stride_h, stride_w,
                        dilation_h, dilation_w, pad_top, pad_left, has_bias, is_depthwise, y_cs, y_cn, y_gs, wrap32,
                        act, stream);
}

extern "C" size_t cm_conv_w_planes_bytes(uint32_t out_ch, uint32_t in_ch, uint32_t kh, uint32_t kw) {
    using namespace cm;
    if (out_ch == 0 || in_ch == 0 || kh == 0 || kw == 0) return 0;
    return make_planes(out_ch, conv_kp(in_ch, kh, kw), 1, 256).bytes();
}

extern "C" int cm_conv_split_w(const int16_t* w, void* planes, uint32_t out_ch, uint32_t in_ch, uint32_t kh,
                               uint32_t kw, void* stream) {
    using namespace cm;
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    if (out_ch == 0) return CM_OK;
    if (in_ch == 0 || kh == 0 || kw == 0 || kh > 7 || kw > 7) return fail(CM_EINVAL, "conv: weights %ux%ux%u", in_ch, kh, kw);
    if ((uint64_t)in_ch * kh * kw > 32768)
        return fail(CM_EINVAL, "conv: in_ch * kh * kw = %u above 32768", in_ch * kh * kw);
    if (reinterpret_cast<uintptr_t>(planes) & 255) return fail(CM_EALIGN, "conv: weight planes not 256-byte aligned");
    Planes A = make_planes(out_ch, conv_kp(in_ch, kh, kw), 1, 256);
    char* p = static_cast<char*>(planes);
    A.carve(p);
    return conv_split_w(w, A, out_ch, in_ch, kh, kw, as_stream(stream));
}

namespace cm {
namespace {

int conv_planes_run(const int16_t* x, const void* w_planes, const int16_t* bias, int16_t* y, uint32_t batch,
                    uint32_t in_ch, uint32_t in_h, uint32_t in_w, uint32_t out_ch, uint32_t out_h, uint32_t out_w,
                    uint32_t kh, uint32_t kw, uint32_t stride_h, uint32_t stride_w, uint32_t dilation_h,
                    uint32_t dilation_w, uint32_t pad_top, uint32_t pad_left, uint32_t has_bias,
                    uint32_t is_depthwise, uint32_t y_cs, uint32_t y_cn, uint32_t y_gs, uint32_t wrap32,
                    uint32_t act, void* stream) {
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    int32_t lo, hi;
    rc = act_bounds(act, lo, hi);
    if (rc) return rc;
    if (batch == 0 || out_ch == 0 || out_h == 0 || out_w == 0) return CM_OK;
    if (is_depthwise) return fail(CM_EINVAL, "conv: weight planes are for standard convolutions");
    if (kh == 0 || kw == 0 || kh > 7 || kw > 7) return fail(CM_EINVAL, "conv: kernel %ux%u outside 1..7", kh, kw);
    if (stride_h == 0 || stride_w == 0 || dilation_h == 0 || dilation_w == 0)
        return fail(CM_EINVAL, "conv: zero stride or dilation");
    if ((y_cs || y_cn) && batch != 1) return fail(CM_EINVAL, "conv: y pattern needs batch 1");
    if (in_ch == 0) return fail(CM_EINVAL, "conv: in_ch 0");
    if ((uint64_t)in_ch * kh * kw > 32768)
        return fail(CM_EINVAL, "conv: in_ch * kh * kw = %u above 32768", in_ch * kh * kw);
    if (reinterpret_cast<uintptr_t>(w_planes) & 255) return fail(CM_EALIGN, "conv: weight planes not 256-byte aligned");
    hipStream_t s = as_stream(stream);
    const uint32_t plane = out_h * out_w;
    const ConvGeom g{batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, stride_h, stride_w, dilation_h,
                     dilation_w, pad_top, pad_left, y_cs ? y_cs : plane, y_cn, y_gs, wrap32 ? 1u : 0u};
    const uint32_t kp = conv_kp(in_ch, kh, kw);
    Planes B = conv_b_planes(g, kp);
    Planes A = make_planes(out_ch, kp, 1, 256);
    char* q = static_cast<char*>(const_cast<void*>(w_planes));
    A.carve(q);
    A.tile = conv_tile(g, B, st);
    void* ws;
    rc = workspace(st, B.bytes(), &ws, s);
    if (rc) return rc;
    char* p = static_cast<char*>(ws);
    B.carve(p);
    return conv_gemm(x, A, B, has_bias ? bias : nullptr, y, g, st, s, lo, hi);
}

}  // namespace
}  // namespace cm

extern "C" int cm_conv_planes(const int16_t* x, const void* w_planes, const int16_t* bias, int16_t* y,
                              uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w, uint32_t out_ch,
                              uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw, uint32_t stride_h,
                              uint32_t stride_w, uint32_t dilation_h, uint32_t dilation_w, uint32_t pad_top,
                              uint32_t pad_left, uint32_t has_bias, uint32_t is_depthwise, uint32_t y_cs,
                              uint32_t y_cn, uint32_t y_gs, uint32_t wrap32, void* stream) {
    return cm::conv_planes_run(x, w_planes, bias, y, batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, stride_h,
                               stride_w, dilation_h, dilation_w, pad_top, pad_left, has_bias, is_depthwise, y_cs,
                               y_cn, y_gs, wrap32, 0, stream);
}

extern "C" int cm_conv_planes_act(const int16_t* x, const void* w_planes, const int16_t* bias, int16_t* y,
                                  uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w, uint32_t out_ch,
                                  uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw, uint32_t stride_h,
                                  uint32_t stride_w, uint32_t dilation_h, uint32_t dilation_w, uint32_t pad_top,
                                  uint32_t pad_left, uint32_t has_bias, uint32_t is_depthwise, uint32_t y_cs,
                                  uint32_t y_cn, uint32_t y_gs, uint32_t wrap32, uint32_t act, void* stream) {
    return cm::conv_planes_run(x, w_planes, bias, y, batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, stride_h,
                               stride_w, dilation_h, dilation_w, pad_top, pad_left, has_bias, is_depthwise, y_cs,
                               y_cn, y_gs, wrap32, act, stream);
}

extern "C" int cm_matmul_strided(const int16_t* a, const int16_t* b, int16_t* c, uint32_t n, uint32_t k, uint32_t m,
                                 uint32_t batch, uint32_t inner, uint64_t lda, uint64_t a_bs, uint64_t a_bs2,
                                 uint64_t ldb, uint64_t b_bs, uint64_t b_bs2, uint32_t b_trans, uint64_t ldc,
                                 uint64_t c_bs, uint64_t c_bs2, uint32_t wrap32, void* stream) {
    using namespace cm;
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    if (n == 0 || m == 0 || batch == 0) return CM_OK;
    if (k == 0 || k > 32768) return fail(CM_EINVAL, "matmul: k = %u outside 1 .. 32768", k);
    if (inner == 0) return fail(CM_EINVAL, "matmul: inner 0");
    const bool a_ok = aligned16(a) && (lda & 7) == 0 && (a_bs & 7) == 0 && (a_bs2 & 7) == 0 && (k & 7) == 0;
    const bool b_ok = aligned16(b) && (ldb & 7) == 0 && (b_bs & 7) == 0 && (b_bs2 & 7) == 0 &&
                      (b_trans ? (k & 7) == 0 : (m & 7) == 0);
    if (!a_ok || !b_ok) return fail(CM_EALIGN, "matmul: strided operands need 16-byte rows and slices");
    if (lda < k || ldb < (b_trans ? k : m) || ldc < m) return fail(CM_EINVAL, "matmul: row strides below the rows");
    hipStream_t s = as_stream(stream);
    const uint32_t kp = (uint32_t)round_up(k, BK);
    Planes A = make_planes(n, kp, batch, gemm_tile_rows(n, m, batch, st->cus)), B = make_planes(m, kp, batch);
    void* ws;
    rc = workspace(st, A.bytes() + B.bytes(), &ws, s);
    if (rc) return rc;
    char* p = static_cast<char*>(ws);
    A.carve(p);
    B.carve(p);
    rc = split_row_lines(a, Slices{a_bs, a_bs2, inner}, lda, n, k, A, s);
    if (rc) return rc;
    if (b_trans) {
        rc = split_row_lines(b, Slices{b_bs, b_bs2, inner}, ldb, m, k, B, s);
        if (rc) return rc;
    } else {
        CM_LAUNCH("split_cols_kernel", split_cols_kernel, dim3(B.lines_p / 32, B.nslab, B.slices), dim3(256), 0, s,
                  b, (Slices{b_bs, b_bs2, inner}), ldb, 0u, m, k, B.hi, B.lo, B.part, B.lines_p, B.kp, B.nslab);
    }
    const bool pairs = (reinterpret_cast<uintptr_t>(c) & 3) == 0 && (m & 1) == 0 && (ldc & 1) == 0 &&
                       (c_bs & 1) == 0 && (c_bs2 & 1) == 0;
    EpiMatmul epi{c, c_bs, n, m, wrap32 ? 1u : 0u, pairs ? 1u : 0u, ldc, c_bs2, inner};
    return run_gemm(A, B, batch, k, epi, s);
}

extern "C" int cm_matmul_skinny_multi(const int16_t* a, uint32_t n, uint32_t k, uint32_t count,
                                      const int16_t* const* b, int16_t* const* c, const uint32_t* m,
                                      uint32_t b_packed, void* stream) {
    using namespace cm;
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    if (count == 0 || count > kSkinnySegs) return fail(CM_EINVAL, "matmul: %u products (1 .. %u)", count, kSkinnySegs);
    if (n == 0) return CM_OK;
    if (n > 32 || k == 0 || k > 32768 || (k & 1) || b_packed > 2 || (b_packed == 2 && (k & 7)))
        return fail(CM_EINVAL, "matmul: skinny products take n <= 32, even k <= 32768 (k %% 8 == 0 transposed)");
    if (reinterpret_cast<uintptr_t>(a) & 3) return fail(CM_EALIGN, "matmul: a not 4-byte aligned");
    for (uint32_t i = 0; i < count; i++) {
        if (m[i] == 0 || (m[i] & 1) || (b_packed == 1 && (m[i] & 31)))
            return fail(CM_EINVAL, "matmul: product %u: m = %u", i, m[i]);
        if ((reinterpret_cast<uintptr_t>(b[i]) & (b_packed == 2 ? 15 : 3)) || (reinterpret_cast<uintptr_t>(c[i]) & 3))
            return fail(CM_EALIGN, "matmul: product %u: b / c not aligned", i);
    }
    return skinny_run(a, n, k, 1, 0, 0, 0, count, b, c, m, b_packed, st, as_stream(stream));
}

namespace cm {
namespace {

// 16-column blocks a skinny workgroup owns, for a launch of blocks16 blocks over k.
uint32_t skinny_blocks(uint64_t blocks16, uint32_t k) {
    (void)k;
    return blocks16 >= 2048 ? 4u : (blocks16 >= 256 ? 2u : 1u);
}

// The segments of a skinny launch (checked, the planes carved), the slabs of their column sums
// and the 16-column blocks they hold.
int skinny_segs(uint32_t n, uint32_t k, uint32_t count, const int16_t* a, const void* const* b_planes,
                int16_t* const* c, const uint32_t* m, SkinnyPlaneSegs& segs, uint32_t& nslab, uint64_t& blocks16) {
    if (count == 0 || count > kSkinnySegs) return fail(CM_EINVAL, "matmul: %u products (1 .. %u)", count, kSkinnySegs);
    if (n > 16 || k == 0 || k > 32768 || (k & 7))
        return fail(CM_EINVAL, "matmul: skinny plane products take n <= 16 and k a multiple of 8 up to 32768");
    if (!aligned16(a)) return fail(CM_EALIGN, "matmul: a not 16-byte aligned");
    const uint32_t kp = (uint32_t)round_up(k, BK);
    segs = SkinnyPlaneSegs{};
    segs.count = count;
    blocks16 = 0;
    nslab = 0;
    for (uint32_t i = 0; i < count; i++) {
        if (m[i] == 0) return fail(CM_EINVAL, "matmul: product %u: m = 0", i);
        if (reinterpret_cast<uintptr_t>(b_planes[i]) & 255)
            return fail(CM_EALIGN, "matmul: product %u: b planes not 256-byte aligned", i);
        Planes B = make_planes(m[i], kp, 1);
        char* q = static_cast<char*>(const_cast<void*>(b_planes[i]));
        B.carve(q);
        segs.hi[i] = B.hi;
        segs.lo[i] = B.lo;
        segs.part[i] = B.part;
        segs.c[i] = c[i];
        segs.m[i] = m[i];
        segs.lines_p[i] = B.lines_p;
        nslab = B.nslab;
        blocks16 += ceil_div(m[i], 16);
    }
    return CM_OK;
}

// Wavefronts of an nb-block skinny workgroup over k (one round of loads where they allow) and
// the LDS of their partials.
uint32_t skinny_waves(uint32_t k, uint32_t nb) {
    const uint32_t kp = (uint32_t)round_up(k, BK);
    return std::min<uint32_t>(sp_max_waves(nb), std::max<uint32_t>(1, ceil_div(kp / 64, sp_chunk(nb))));
}
size_t skinny_lds(uint32_t waves, uint32_t nb, bool sat = false) {
    return (size_t)waves * 16 * (16 * nb * (sat ? 3 : 1) + 1) * 4;
}

int skinny_planes(const int16_t* a, uint32_t n, uint32_t k, uint32_t count, const void* const* b_planes,
                  int16_t* const* c, const uint32_t* m, const SkinnyAddx& ax, hipStream_t s, bool sat = false) {
    if (n == 0) return CM_OK;
    SkinnyPlaneSegs segs;
    uint32_t nslab;
    uint64_t blocks16;
    int rc = skinny_segs(n, k, count, a, b_planes, c, m, segs, nslab, blocks16);
    if (rc) return rc;
    const uint32_t kp = (uint32_t)round_up(k, BK);
    // the saturating partials take three times the LDS: at most two blocks a workgroup (50 KiB)
    const uint32_t nb = sat ? std::min<uint32_t>(2, skinny_blocks(blocks16, k)) : skinny_blocks(blocks16, k);
    uint64_t cbs = 0;
    for (uint32_t i = 0; i < count; i++) {
        segs.cb0[i] = (uint32_t)cbs;
        cbs += ceil_div(m[i], 16 * nb);
    }
    if (cbs > 0x7FFFFFFFull) return fail(CM_EINVAL, "matmul: %llu column blocks", (unsigned long long)cbs);
    const uint32_t waves = skinny_waves(k, nb);
    const size_t lds = skinny_lds(waves, nb, sat);
    const dim3 grid((uint32_t)cbs), block(64 * waves);
    const uint32_t xk = ax.out == nullptr ? 0u : (((ax.op >> 4) & 3) == 0 ? 1u : 2u);
    if (sat && xk) return fail(CM_EINVAL, "matmul: no output job on saturating skinny products");
#define CM_SP_LAUNCH(NB_, XK_)                                                                                  \
    CM_LAUNCH("skinny_planes_kernel", (skinny_planes_kernel<NB_, XK_>), grid, block, lds, s, a, n, k, kp, nslab, \
              segs, ax)
#define CM_SP_LAUNCH_SAT(NB_)                                                                                   \
    CM_LAUNCH("skinny_planes_kernel", (skinny_planes_kernel<NB_, 0, true>), grid, block, lds, s, a, n, k, kp,    \
              nslab, segs, ax)
    if (sat) {
        if (nb == 1) { CM_SP_LAUNCH_SAT(1); }
        else { CM_SP_LAUNCH_SAT(2); }
    } else if (xk == 0) {
        if (nb == 1) { CM_SP_LAUNCH(1, 0); }
        else if (nb == 2) { CM_SP_LAUNCH(2, 0); }
        else { CM_SP_LAUNCH(4, 0); }
    } else if (xk == 1) {
        if (nb == 1) { CM_SP_LAUNCH(1, 1); }
        else if (nb == 2) { CM_SP_LAUNCH(2, 1); }
        else { CM_SP_LAUNCH(4, 1); }
    } else {
        if (nb == 1) { CM_SP_LAUNCH(1, 2); }
        else if (nb == 2) { CM_SP_LAUNCH(2, 2); }
        else { CM_SP_LAUNCH(4, 2); }
    }
#undef CM_SP_LAUNCH
#undef CM_SP_LAUNCH_SAT
    return CM_OK;
}

int skinny_mulact(const int16_t* a, uint32_t n, uint32_t k, const void* b_gate, const void* b_up, int16_t* c_gate,
                  int16_t* c_up, uint32_t m, const SkinnyMulact& mj, hipStream_t s) {
    if (n == 0) return CM_OK;
    SkinnyPlaneSegs segs;
    uint32_t nslab;
    uint64_t blocks16;
    const void* bp[2] = {b_gate, b_up};
    int16_t* cp[2] = {c_gate, c_up};
    const uint32_t ms[2] = {m, m};
    int rc = skinny_segs(n, k, 2, a, bp, cp, ms, segs, nslab, blocks16);
    if (rc) return rc;
    (void)blocks16;
    const uint32_t kp = (uint32_t)round_up(k, BK);
    const uint32_t waves = skinny_waves(k, 2);      // 16 gate and 16 up columns a workgroup
    CM_LAUNCH("skinny_mulact_kernel", skinny_mulact_kernel<2>, dim3(ceil_div(m, 16)), dim3(64 * waves),
              skinny_lds(waves, 2), s, a, n, k, kp, nslab, segs, mj);
    return CM_OK;
}

}  // namespace
}  // namespace cm

extern "C" int cm_matmul_skinny_planes_mulact(const int16_t* a, uint32_t n, uint32_t k, const void* b_gate,
                                              const void* b_up, int16_t* c_gate, int16_t* c_up, uint32_t m,
                                              const void* params, uint32_t op, int16_t* out, void* stream) {
    using namespace cm;
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    if ((op & 15) != ro::RO_MULACT || !(op & ro::F_B_EN) || (op & ro::F_P_KEEP) || ((op >> 4) & 3) != 0 ||
        ((op >> 6) & 3) != 0 || ((op >> 8) & 3) != 0)
        return fail(CM_EINVAL, "matmul: the output job must be an int16 MULACT with B enabled (op 0x%x)", op);
    if (params == nullptr || out == nullptr || c_gate == nullptr || c_up == nullptr)
        return fail(CM_EINVAL, "matmul: the MULACT output needs both products, out and a parameter block");
    if (m > ro::kNMax) return fail(CM_EINVAL, "matmul: the MULACT job's rows of %u above %u", m, ro::kNMax);
    if ((reinterpret_cast<uintptr_t>(params) & 15) || (reinterpret_cast<uintptr_t>(out) & 1) ||
        (reinterpret_cast<uintptr_t>(c_gate) & 1) || (reinterpret_cast<uintptr_t>(c_up) & 1))
        return fail(CM_EALIGN, "matmul: the MULACT operands are not aligned");
    const SkinnyMulact mj{out, static_cast<const uint8_t*>(params), (op & ro::F_P_BCAST) ? 1u : 0u, st->ro_tables};
    return skinny_mulact(a, n, k, b_gate, b_up, c_gate, c_up, m, mj, as_stream(stream));
}

extern "C" int cm_matmul_skinny_planes(const int16_t* a, uint32_t n, uint32_t k, uint32_t count,
                                       const void* const* b_planes, int16_t* const* c, const uint32_t* m,
                                       void* stream) {
    using namespace cm;
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    return skinny_planes(a, n, k, count, b_planes, c, m, SkinnyAddx{}, as_stream(stream));
}

extern "C" int cm_matmul_skinny_planes_sat(const int16_t* a, uint32_t n, uint32_t k, uint32_t count,
                                           const void* const* b_planes, int16_t* const* c, const uint32_t* m,
                                           void* stream) {
    using namespace cm;
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    return skinny_planes(a, n, k, count, b_planes, c, m, SkinnyAddx{}, as_stream(stream), true);
}

extern "C" int cm_matmul_skinny_planes_addx(const int16_t* a, uint32_t n, uint32_t k, const void* b_planes,
                                            int16_t* c, uint32_t m, const void* x, const void* params, uint32_t op,
                                            uint32_t bq_sh, void* out, void* stream) {
    using namespace cm;
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    const uint32_t code = op & 15, ak = (op >> 4) & 3, bk = (op >> 6) & 3, ck = (op >> 8) & 3;
    if ((code != ro::RO_COPY && code != ro::RO_ADDX) || !(op & ro::F_B_EN) || (op & ro::F_P_KEEP) || ak > 1 ||
        bk != 0 || ck > 1 || bq_sh > 63)
        return fail(CM_EINVAL, "matmul: the output job must be a COPY / ADDX with B the int16 product (op 0x%x)", op);
    if (x == nullptr || out == nullptr || params == nullptr)
        return fail(CM_EINVAL, "matmul: the output job needs x, out and a parameter block");
    if ((reinterpret_cast<uintptr_t>(x) & (ak ? 3 : 1)) || (reinterpret_cast<uintptr_t>(out) & (ck ? 3 : 1)) ||
        (reinterpret_cast<uintptr_t>(params) & 15))
        return fail(CM_EALIGN, "matmul: the output job's operands are not aligned");
    const SkinnyAddx ax{static_cast<const uint8_t*>(x), static_cast<uint8_t*>(out), static_cast<const uint8_t*>(params),
                        op, bq_sh};
    return skinny_planes(a, n, k, 1, &b_planes, &c, &m, ax, as_stream(stream));
}
