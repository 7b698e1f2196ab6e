// Accent adapter shift of a projection: y_out = y_in + ((x . down^T) * mask) . up, per row, with the
// rounding points of the reference's bf16 torch ops (servers/sgl/src/zonos3_sgl/layers/accent.py:25-62:
// x @ down.T rounded, times mask rounded, @ up rounded, added to y rounded).
//
// Two launches. accent_down_kernel forms tm = round(round(x . down^T) * mask) [rows, Kp] (Kp = K rounded up
// to 32, zero columns past K) into a small workspace, and with a few more workgroups up^T [out, Kp];
// accent_up_kernel streams y: each workgroup forms y_out = y_in + round(tm . up) for 64 rows x 128 columns
// (y_out may be y_in). Both run on
// bf16 MFMA (v_mfma_f32_16x16x32_bf16, fp32 accumulation) for bf16; fp32 runs plain fp32 arithmetic.
// Every row is computed on its own in a fixed order, so a row's result never depends on the other rows of
// the call (the batch invariance the reference gets by padding to fixed-row blocks).
#include <algorithm>
#include <type_traits>

#include "gdn_common.h"

namespace zgdn {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int AC_ROWS = 64;   // rows per workgroup (16 per wave)
constexpr int AC_NB = 128;    // output columns per phase-2 workgroup
constexpr int AC_KMAX = 256;  // adapter columns (sum of the loaded adapters' ranks)

__device__ __forceinline__ int kpad(int K) { return (K + 31) / 32 * 32; }

__device__ __forceinline__ float rbf(float x) { return bf16_to_f32(f32_to_bf16(x)); }

__device__ __forceinline__ f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 load8(const uint16_t* p, bool ok) {
  const uint4 w = ok ? *reinterpret_cast<const uint4*>(p) : make_uint4(0, 0, 0, 0);
  return __builtin_bit_cast(bf16x8, w);
}

// tm[r][k] = round(round(sum_i x[r][i] down[k][i]) * mask[r][k]) for 16 rows per workgroup and every k < Kp.
// Wave w sums the inputs i in its quarter of [0, in) (32 at a time, MFMA D tiles of 16 rows x 16 columns k:
// lane holds rows 4 (l / 16) + j, column l % 16); the four partial tiles are added in wave order through
// LDS, the same order for every row.
// Workgroups past the row blocks write up^T [out][Kp] (zero columns past K) for the second kernel, 64 output
// columns each, through an LDS transpose.
__device__ __forceinline__ void transpose_up(const uint16_t* __restrict__ up, uint16_t* __restrict__ upT,
                                             int out, int K, int n0, uint16_t* tile) {
  const int Kp = kpad(K), pitch = Kp + 8, tid = threadIdx.x;
  for (int e = tid; e < Kp * 8; e += 256) {  // row k, columns n0 + 8 (e % 8) .. +7
    const int k = e / 8, c8 = (e % 8) * 8;
    const bool ok = k < K && n0 + c8 < out;  // out is a multiple of 8
    const uint4 w = ok ? *reinterpret_cast<const uint4*>(up + (size_t)k * out + n0 + c8) : make_uint4(0, 0, 0, 0);
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      tile[(c8 + 2 * j) * pitch + k] = (uint16_t)(u[j] & 0xffffu);
      tile[(c8 + 2 * j + 1) * pitch + k] = (uint16_t)(u[j] >> 16);
    }
  }
  __syncthreads();
  for (int e = tid; e < 64 * (Kp / 8); e += 256) {  // row n0 + n of up^T, keys 8 (e % (Kp / 8)) .. +7
    const int n = e / (Kp / 8), k8 = (e % (Kp / 8)) * 8;
    if (n0 + n < out)
      *reinterpret_cast<uint4*>(upT + (size_t)(n0 + n) * Kp + k8) = *reinterpret_cast<const uint4*>(&tile[n * pitch + k8]);
  }
}

template <int NT>
__global__ __launch_bounds__(256) void accent_down_bf16_kernel(const uint16_t* __restrict__ x, long x_ld,
                                                               const uint16_t* __restrict__ down,
                                                               const uint16_t* __restrict__ mask, long mask_ld,
                                                               uint16_t* __restrict__ tm, const uint16_t* __restrict__ up,
                                                               uint16_t* __restrict__ upT, int rows, int in, int out,
                                                               int K) {
  __shared__ f32x4 part[4][NT][64];  // also the transpose tile (64 x (Kp + 8) bf16 <= 4 x NT x 64 x 16 bytes)
  const int Kp = kpad(K);
  const int n_row_blocks = (rows + 15) / 16;
  if ((int)blockIdx.x >= n_row_blocks) {
    transpose_up(up, upT, out, K, ((int)blockIdx.x - n_row_blocks) * 64, reinterpret_cast<uint16_t*>(part));
    return;
  }
  const int l = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r0 = blockIdx.x * 16;
  const int ra = r0 + (l & 15);
  const bool row_ok = ra < rows;
  const int steps = (in + 31) / 32, per = (steps + 3) / 4;
  const int s0 = wave * per, s1 = min(steps, s0 + per);
  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int st = s0; st < s1; ++st) {
    const int i = 32 * st + 8 * (l >> 4);
    const bf16x8 a = load8(x + (size_t)ra * x_ld + i, row_ok && i < in);
    bf16x8 b[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int k = 16 * t + (l & 15);
      b[t] = load8(down + (size_t)k * in + i, 16 * t < Kp && k < K && i < in);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t)
      if (16 * t < Kp) acc[t] = mfma_bf16(a, b[t], acc[t]);
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) part[wave][t][l] = acc[t];
  __syncthreads();
  // wave w finishes tiles t = w, w + 4, ...
  for (int t = wave; t < NT; t += 4) {
    if (16 * t >= Kp) break;
    const f32x4 sum = ((part[0][t][l] + part[1][t][l]) + part[2][t][l]) + part[3][t][l];
    const int k = 16 * t + (l & 15);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = r0 + 4 * (l >> 4) + j;
      if (r >= rows) continue;
      const float m = k < K ? bf16_to_f32(mask[(size_t)r * mask_ld + k]) : 0.f;
      tm[(size_t)r * Kp + k] = f32_to_bf16(rbf(sum[j]) * m);
    }
  }
}

// y_out[r][n] = round(y_in[r][n] + round(sum_k tm[r][k] up[k][n])) for AC_RB blocks of 64 rows x 128 columns.
// The workgroup copies its 128 rows of up^T into LDS once and walks its row blocks with the next block's y_in
// loads in flight (16 bytes = 8 columns of one row per load, whole rows per instruction). Per block it forms
// the products on MFMA with the output columns as the M side (A = up^T from LDS) and the rows as the N side
// (B = tm rows), rounds them to bf16 through LDS in row order and adds them to its y values: every y access is
// 16 contiguous bytes.
constexpr int AC_RB = 2;  // 64-row blocks per phase-2 workgroup (the sweep over 1, 2, 4, 8: 2 best)
template <bool HAS_Y, bool ALIGNED>
__global__ __launch_bounds__(256) void accent_up_bf16_kernel(const uint16_t* __restrict__ tm,
                                                             const uint16_t* __restrict__ upT,
                                                             const uint16_t* y_in, long y_in_ld,
                                                             uint16_t* y_out, long y_out_ld, int rows,
                                                             int out, int K) {  // y_out may equal y_in
  constexpr int NB = AC_NB, SP = NB + 8;
  extern __shared__ uint16_t lds[];  // up^T tile [NB][Kp + 8], then the products [AC_ROWS][SP]
  const int Kp = kpad(K), pitch = Kp + 8;
  uint16_t* ut = lds;
  uint16_t* sh = lds + NB * pitch;
  // Workgroup ids go round-robin over the 8 XCDs: all column blocks of one row block take ids of one residue
  // mod 8, so they run on one XCD and share its L2 copy of the 128-byte lines their rows straddle (the
  // projection's rows are rarely line-aligned: 2056 bf16 = 4112 bytes).
  const int n_nb = (out + NB - 1) / NB, n_rb = (rows + AC_ROWS * AC_RB - 1) / (AC_ROWS * AC_RB);
  const int xcd = blockIdx.x % 8, slot = blockIdx.x / 8;
  const int rblk = (slot / n_nb) * 8 + xcd, nblk = slot % n_nb;
  if (rblk >= n_rb) return;
  const int n0 = nblk * NB, rbase = rblk * (AC_ROWS * AC_RB);
  const int tid = threadIdx.x, l = tid & 63, wave = tid >> 6;
  constexpr int G = NB / 8;               // 16-byte groups per row of y
  constexpr int PER = AC_ROWS * G / 256;  // y groups per thread and block
  auto load_y = [&](int r0, uint4* yw) {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int e = tid + 256 * p, r = r0 + e / G, n = n0 + 8 * (e % G);
      yw[p] = make_uint4(0, 0, 0, 0);
      if (HAS_Y && r < rows && n < out) {
        const uint16_t* yp = y_in + (size_t)r * y_in_ld + n;
        if constexpr (ALIGNED) {
          yw[p] = *reinterpret_cast<const uint4*>(yp);
        } else {
          uint32_t u[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) u[j] = (uint32_t)yp[2 * j] | ((uint32_t)yp[2 * j + 1] << 16);
          yw[p] = make_uint4(u[0], u[1], u[2], u[3]);
        }
      }
    }
  };
  uint4 ya[PER], yb[PER];
  load_y(rbase, ya);
  for (int e = tid; e < NB * (Kp / 8); e += 256) {  // up^T rows n0 .. n0 + NB - 1 into LDS
    const int n = e / (Kp / 8), k8 = (e % (Kp / 8)) * 8;
    const uint4 w = n0 + n < out ? *reinterpret_cast<const uint4*>(upT + (size_t)(n0 + n) * Kp + k8)
                                 : make_uint4(0, 0, 0, 0);
    *reinterpret_cast<uint4*>(&ut[n * pitch + k8]) = w;
  }
  __syncthreads();

  constexpr int NT = NB / 16;
  auto block = [&](int r0, const uint4* yw) {
    // wave w: rows r0 + 16 w .. +15 (MFMA N side), all NB columns
    const int rb = r0 + 16 * wave + (l & 15);
    f32x4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < Kp; k0 += 32) {
      const int kk = k0 + 8 * (l >> 4);
      const bf16x8 b = load8(tm + (size_t)rb * Kp + kk, rb < rows);
#pragma unroll
      for (int t = 0; t < NT; ++t)
        acc[t] = mfma_bf16(*reinterpret_cast<const bf16x8*>(&ut[(16 * t + (l & 15)) * pitch + kk]), b, acc[t]);
    }
    // D: lane holds columns 16 t + 4 (l / 16) + j of row 16 w + l % 16: rounded products to LDS
    const int rr = 16 * wave + (l & 15);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int c = 16 * t + 4 * (l >> 4);
      *reinterpret_cast<uint2*>(&sh[rr * SP + c]) =
          make_uint2(pack_bf16x2(acc[t][0], acc[t][1]), pack_bf16x2(acc[t][2], acc[t][3]));
    }
    __syncthreads();
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int e = tid + 256 * p, rl = e / G, cl = 8 * (e % G), r = r0 + rl, n = n0 + cl;
      if (r >= rows || n >= out) continue;
      const uint4 sw = *reinterpret_cast<const uint4*>(&sh[rl * SP + cl]);
      const uint32_t su[4] = {sw.x, sw.y, sw.z, sw.w}, yu[4] = {yw[p].x, yw[p].y, yw[p].z, yw[p].w};
      uint32_t ou[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float s_lo = __uint_as_float(su[j] << 16), s_hi = __uint_as_float(su[j] & 0xffff0000u);
        const float y_lo = __uint_as_float(yu[j] << 16), y_hi = __uint_as_float(yu[j] & 0xffff0000u);
        ou[j] = HAS_Y ? pack_bf16x2(y_lo + s_lo, y_hi + s_hi) : su[j];
      }
      uint16_t* op = y_out + (size_t)r * y_out_ld + n;
      if constexpr (ALIGNED) {
        *reinterpret_cast<uint4*>(op) = make_uint4(ou[0], ou[1], ou[2], ou[3]);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          op[2 * j] = (uint16_t)(ou[j] & 0xffffu);
          op[2 * j + 1] = (uint16_t)(ou[j] >> 16);
        }
      }
    }
    __syncthreads();  // the products' LDS is rewritten by the next block
  };
  // blocks alternate between the two y buffers, the next block's loads issued before the current one's work
#pragma unroll
  for (int b = 0; b < AC_RB; b += 2) {
    const int r0 = rbase + AC_ROWS * b;
    if (r0 >= rows) break;
    load_y(r0 + AC_ROWS, yb);
    block(r0, ya);
    if (r0 + AC_ROWS >= rows) break;
    if (b + 2 < AC_RB) load_y(r0 + 2 * AC_ROWS, ya);
    block(r0 + AC_ROWS, yb);
  }
}

// fp32: one thread per (row, adapter column) / (row, output column), fp32 throughout.
__global__ __launch_bounds__(256) void accent_down_f32_kernel(const float* __restrict__ x, long x_ld,
                                                              const float* __restrict__ down,
                                                              const float* __restrict__ mask, long mask_ld,
                                                              float* __restrict__ tm, int rows, int in, int K) {
  const int Kp = kpad(K);
  const long e = (long)blockIdx.x * 256 + threadIdx.x;
  if (e >= (long)rows * Kp) return;
  const int r = (int)(e / Kp), k = (int)(e % Kp);
  float acc = 0.f;
  if (k < K) {
    for (int i = 0; i < in; ++i) acc = fmaf(x[(size_t)r * x_ld + i], down[(size_t)k * in + i], acc);
    acc *= mask[(size_t)r * mask_ld + k];
  }
  tm[(size_t)r * Kp + k] = acc;
}

__global__ __launch_bounds__(256) void accent_up_f32_kernel(const float* __restrict__ tm, const float* __restrict__ up,
                                                            const float* y_in, long y_in_ld, float* y_out,
                                                            long y_out_ld, int rows, int out, int K) {
  const int Kp = kpad(K);
  const long e = (long)blockIdx.x * 256 + threadIdx.x;
  if (e >= (long)rows * out) return;
  const int r = (int)(e / out), n = (int)(e % out);
  float acc = 0.f;
  for (int k = 0; k < K; ++k) acc = fmaf(tm[(size_t)r * Kp + k], up[(size_t)k * out + n], acc);
  y_out[(size_t)r * y_out_ld + n] = (y_in != nullptr ? y_in[(size_t)r * y_in_ld + n] : 0.f) + acc;
}

}  // namespace
}  // namespace zgdn

extern "C" size_t zgdn_accent_workspace_size(int rows, int out, int K, int dtype) {
  if (rows <= 0 || out <= 0 || K <= 0) return 0;
  const size_t Kp = (size_t)((K + 31) / 32 * 32);
  // tm [rows, Kp]; bf16 also up^T [out, Kp]
  return dtype == ZGDN_F32 ? (size_t)rows * Kp * 4 : ((size_t)rows + (size_t)out) * Kp * 2;
}

extern "C" int zgdn_accent_shift(const void* x, long x_ld, const void* down, const void* up, const void* mask,
                                 long mask_ld, const void* y_in, long y_in_ld, void* y_out, long y_out_ld, int rows,
                                 int in, int out, int K, int dtype, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  using namespace zgdn;
  const char* fn = "zgdn_accent_shift";
  if (!x || !down || !up || !mask || !y_out || !workspace) return fail(ZGDN_EINVAL, "%s: null pointer", fn);
  if (dtype != ZGDN_F32 && dtype != ZGDN_BF16) return fail(ZGDN_EINVAL, "%s: dtype code %d", fn, dtype);
  if (rows < 0 || in < 1 || out < 1 || K < 1 || K > AC_KMAX)
    return fail(ZGDN_EUNSUPPORTED, "%s: rows=%d in=%d out=%d K=%d (K <= %d)", fn, rows, in, out, K, AC_KMAX);
  if (x_ld < in || mask_ld < K || y_out_ld < out || (y_in != nullptr && y_in_ld < out))
    return fail(ZGDN_EINVAL, "%s: row strides x=%ld mask=%ld y_in=%ld y_out=%ld below the row widths", fn, x_ld,
                mask_ld, y_in_ld, y_out_ld);
  const bool bf = dtype == ZGDN_BF16;
  if (bf && (in % 8 || out % 8 || x_ld % 8 || ((uintptr_t)x | (uintptr_t)down | (uintptr_t)up) % 16))
    return fail(ZGDN_EINVAL, "%s: bf16 needs in, out and the x row stride multiples of 8 and 16-byte aligned x, "
                "down, up (in=%d out=%d x_ld=%ld)", fn, in, out, x_ld);
  if (bf && (uintptr_t)workspace % 16) return fail(ZGDN_EINVAL, "%s: workspace not 16-byte aligned", fn);
  if (workspace_bytes < zgdn_accent_workspace_size(rows, out, K, dtype))
    return fail(ZGDN_EINVAL, "%s: workspace of %zu bytes, need %zu", fn, workspace_bytes,
                zgdn_accent_workspace_size(rows, out, K, dtype));
  if (rows == 0) return check_launch(fn);
  hipStream_t s = (hipStream_t)stream;
  const int Kp = (K + 31) / 32 * 32;
  if (bf) {
    // row blocks of 16, then one workgroup per 64 output columns writing up^T
    const dim3 g1((rows + 15) / 16 + (out + 63) / 64);
    auto d = (const uint16_t*)down;
    auto m = (const uint16_t*)mask;
    auto tm = (uint16_t*)workspace;
    auto upT = tm + (size_t)rows * Kp;
    auto go1 = [&](auto nt) {
      constexpr int NT = decltype(nt)::value;  // MFMA column tiles per wave, Kp / 16 rounded up to a power of 2
      hipLaunchKernelGGL(accent_down_bf16_kernel<NT>, g1, dim3(256), 0, s, (const uint16_t*)x, x_ld, d, m, mask_ld,
                         tm, (const uint16_t*)up, upT, rows, in, out, K);
    };
    if (Kp <= 32) go1(std::integral_constant<int, 2>{});
    else if (Kp <= 64) go1(std::integral_constant<int, 4>{});
    else if (Kp <= 128) go1(std::integral_constant<int, 8>{});
    else go1(std::integral_constant<int, 16>{});
    const bool aligned = (((uintptr_t)y_out | (uintptr_t)(y_in ? y_in : y_out)) % 16 == 0) && y_out_ld % 8 == 0 &&
                         (y_in == nullptr || y_in_ld % 8 == 0);
    const int n_nb = (out + AC_NB - 1) / AC_NB, n_rb = (rows + AC_ROWS * AC_RB - 1) / (AC_ROWS * AC_RB);
    const dim3 g2(8 * n_nb * ((n_rb + 7) / 8));  // XCD-grouped ids (see the kernel)
    const size_t lds = ((size_t)AC_NB * (Kp + 8) + (size_t)AC_ROWS * (AC_NB + 8)) * 2;  // <= 84,992 bytes
    auto up2 = y_in != nullptr ? (aligned ? accent_up_bf16_kernel<true, true> : accent_up_bf16_kernel<true, false>)
                               : (aligned ? accent_up_bf16_kernel<false, true> : accent_up_bf16_kernel<false, false>);
    if (lds > 65536 &&
        hipFuncSetAttribute((const void*)up2, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return fail(ZGDN_EHIP, "%s: %zu bytes of LDS for K=%d not available", fn, lds, K);
    hipLaunchKernelGGL(up2, g2, dim3(256), lds, s, tm, upT, (const uint16_t*)y_in, y_in_ld, (uint16_t*)y_out,
                       y_out_ld, rows, out, K);
  } else {
    auto tm = (float*)workspace;
    const long n1 = (long)rows * Kp, n2 = (long)rows * out;
    hipLaunchKernelGGL(accent_down_f32_kernel, dim3((unsigned)((n1 + 255) / 256)), dim3(256), 0, s, (const float*)x,
                       x_ld, (const float*)down, (const float*)mask, mask_ld, tm, rows, in, K);
    hipLaunchKernelGGL(accent_up_f32_kernel, dim3((unsigned)((n2 + 255) / 256)), dim3(256), 0, s, tm,
                       (const float*)up, (const float*)y_in, y_in_ld, (float*)y_out, y_out_ld, rows, out, K);
  }
  return check_launch(fn);
}
