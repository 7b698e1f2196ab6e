// Full Attention-Residual routing: the mix every GDN / attention / FFN sublayer of the LM reads, and the
// bank its output joins (model/src/zonos3/reference/lm.py:384-389; servers/sgl/src/zonos3_sgl/models/
// zonos3.py:99-113), with the reference's rounding points for a bf16 bank:
//   keys_s   = rms_norm(source_s)                 per token, over dim, no weight; rounded to the dtype
//   logit_s  = sum(keys_s * query)                the products rounded to the dtype, summed in fp32
//   w        = softmax over the sources s         fp32, then rounded to the dtype
//   out      = sum_s w_s * source_s               the products rounded to the dtype, summed in fp32
// Sources are given as separate [tokens, dim] row arrays (no stacked copy of the bank). HBM-bound: every
// source row is read from memory once (the second pass finds it in L2) and the mix written once.
//
// Work layout: a workgroup of AR_WAVES waves per token; wave w takes sources w, w + AR_WAVES, ... in both
// passes, reading each row as 16-byte pieces (lane l holds columns 8 (l + 64 c) .. +7). Pass 1 writes the
// logits to LDS; after a barrier every wave forms the softmax weights from them; pass 2 accumulates its
// sources' weighted rows and the waves' partial sums are added through LDS.
#include "gdn_common.h"

namespace zgdn {
namespace {

constexpr int AR_WAVES = 4;


constexpr int AR_MAX_SOURCES = 64;

struct SourcePtrs {
  const void* p[AR_MAX_SOURCES];
};

template <typename T>
struct row8;  // 8 consecutive elements as floats
template <>
struct row8<bf16> {
  __device__ __forceinline__ static void load(const bf16* p, float* f) {
    const uint4 w = *reinterpret_cast<const uint4*>(p);
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(u[i] << 16);
      f[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
    }
  }
  __device__ __forceinline__ static void store(bf16* p, const float* f) {
    *reinterpret_cast<uint4*>(p) = make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]),
                                              pack_bf16x2(f[4], f[5]), pack_bf16x2(f[6], f[7]));
  }
};
template <>
struct row8<float> {
  __device__ __forceinline__ static void load(const float* p, float* f) {
    const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
  }
  __device__ __forceinline__ static void store(float* p, const float* f) {
    *reinterpret_cast<float4*>(p) = make_float4(f[0], f[1], f[2], f[3]);
    *reinterpret_cast<float4*>(p + 4) = make_float4(f[4], f[5], f[6], f[7]);
  }
};

template <typename T>
__device__ __forceinline__ float round_to_t(float x) {
  if constexpr (sizeof(T) == 2) return bf16_to_f32(f32_to_bf16(x));
  else return x;
}

// Two values rounded to T at once (one packed conversion for bf16).
template <typename T>
__device__ __forceinline__ void round2_t(float& a, float& b) {
  if constexpr (sizeof(T) == 2) {
    const uint32_t p = pack_bf16x2(a, b);
    a = __uint_as_float(p << 16);
    b = __uint_as_float(p & 0xffff0000u);
  }
}

// a.lo * b.lo + a.hi * b.hi + c for two bf16 pairs (v_dot2c_f32_bf16): the products of bf16 values are exact
// in fp32, so with one half of b zero this is an exact product (plus c), and with b = (1, 1) the fp32 sum of
// the two halves of a (plus c).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}
// The 8 rounded products of a piece: out[i] = (round(a[i].lo * lo[i].lo + a[i].hi * lo[i].hi),
// round(a[i].lo * hi[i].lo + a[i].hi * hi[i].hi)) -- with one half of each lo / hi word zero, the exact products
// of the pair's two halves, rounded to bf16 and packed. The products run on the three-operand v_dot2_f32_bf16
// with an inline zero addend (the compiler forms dot2_bf16(a, b, 0.f) as v_dot2c_f32_bf16 on a register it
// zeroes first, one more instruction per product). One block for all 12 instructions, so that a VALU read of a
// dot product's result comes at least 3 instructions after it (the wait states it needs, which the compiler
// does not know for an asm block's results): the first conversion reads products 6 and 7 instructions old,
// the last 3 and 4.
__device__ __forceinline__ void products8(const uint32_t (&a)[4], const uint32_t (&lo)[4], const uint32_t (&hi)[4],
                                          uint32_t (&out)[4]) {
  float t[8];
  asm("v_dot2_f32_bf16 %4, %12, %16, 0\n\t"
      "v_dot2_f32_bf16 %5, %12, %20, 0\n\t"
      "v_dot2_f32_bf16 %6, %13, %17, 0\n\t"
      "v_dot2_f32_bf16 %7, %13, %21, 0\n\t"
      "v_dot2_f32_bf16 %8, %14, %18, 0\n\t"
      "v_dot2_f32_bf16 %9, %14, %22, 0\n\t"
      "v_dot2_f32_bf16 %10, %15, %19, 0\n\t"
      "v_dot2_f32_bf16 %11, %15, %23, 0\n\t"
      "v_cvt_pk_bf16_f32 %0, %4, %5\n\t"
      "v_cvt_pk_bf16_f32 %1, %6, %7\n\t"
      "v_cvt_pk_bf16_f32 %2, %8, %9\n\t"
      "v_cvt_pk_bf16_f32 %3, %10, %11"
      : "=&v"(out[0]), "=&v"(out[1]), "=&v"(out[2]), "=&v"(out[3]), "=&v"(t[0]), "=&v"(t[1]), "=&v"(t[2]),
        "=&v"(t[3]), "=&v"(t[4]), "=&v"(t[5]), "=&v"(t[6]), "=&v"(t[7])
      : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(lo[0]), "v"(lo[1]), "v"(lo[2]), "v"(lo[3]), "v"(hi[0]),
        "v"(hi[1]), "v"(hi[2]), "v"(hi[3]));
}
constexpr uint32_t BF16_ONE_HI = 0x3f800000u, BF16_ONES = 0x3f803f80u;
// (1, 0): bf16 1.0 in the low half, in a register. As an immediate, the compiler encodes this operand as the
// inline constant 1.0, which the instruction reads as the fp32 word 0x3f800000, i.e. (0, 1).
__device__ __forceinline__ uint32_t bf16_one_lo() {
  uint32_t r;
  asm volatile("v_mov_b32 %0, 0x3f80" : "=v"(r));
  return r;
}

// Token of workgroup b, or -1 for none. The dispatcher puts workgroups b, b + n_cu, b + 2 n_cu, ... on one
// CU, so with one token per workgroup in order a CU's concurrent workgroups read rows 2 KiB x n_cu apart in
// each of the ~24 source arrays. With per > 0 (calls of at least n_cu tokens, launched as n_cu x per
// workgroups) CU c walks the contiguous tokens c per .. c per + per - 1 instead, and its reads of each source
// stay on the same pages: 23 sources x 4096 x 1024 took 37.8-38.2 us in every allocation state tried, against
// 38.5-45.1 us in order, whose time followed where the arrays had been placed (translation misses); 4
// adjacent tokens per CU group measured about 39.0 us. per = 0: token b.
__device__ __forceinline__ int cu_local_token(int b, int tokens, int n_cu, int per) {
  const int t = per > 0 ? (b % n_cu) * per + b / n_cu : b;
  return t < tokens ? t : -1;
}

// NCH: 8-element pieces per lane (dim <= 512 NCH); columns past dim are masked.
template <typename T, int NCH>
__global__ __launch_bounds__(64 * AR_WAVES) void attnres_kernel(const SourcePtrs src, int n_sources, int dim,
                                                                  long row_stride, const T* __restrict__ query,
                                                                  float eps, T* __restrict__ out, int tokens,
                                                                  int n_cu, int per) {
  __shared__ float s_acc[AR_WAVES][NCH * 8][64];
  __shared__ float s_logit[AR_MAX_SOURCES];
  const int token = cu_local_token(blockIdx.x, tokens, n_cu, per);
  if (token < 0) return;
  const int lane = threadIdx.x & 63, wave = wave_id();
  bool on[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) on[c] = 8 * (lane + 64 * c) < dim;
  auto load_row = [&](int s, float (&x)[NCH][8]) {
    const T* row = reinterpret_cast<const T*>(src.p[s]) + (size_t)token * row_stride;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (on[c]) row8<T>::load(row + 8 * (lane + 64 * c), x[c]);
      else
        for (int i = 0; i < 8; ++i) x[c][i] = 0.f;
    }
  };

  // pass 1: logits
  float q[NCH][8];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (on[c]) row8<T>::load(query + 8 * (lane + 64 * c), q[c]);
    else
      for (int i = 0; i < 8; ++i) q[c][i] = 0.f;
  }
  const float inv_dim = 1.f / (float)dim;
  for (int s = wave; s < n_sources; s += AR_WAVES) {
    float x[NCH][8], ss = 0.f;
    load_row(s, x);
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = fmaf(x[c][i], x[c][i], ss);
    const float r = rsqrtf(wave_sum(ss) * inv_dim + eps);
    float lg = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int i = 0; i < 8; ++i) lg += round_to_t<T>(round_to_t<T>(x[c][i] * r) * q[c][i]);
    lg = wave_sum(lg);
    if (lane == 0) s_logit[s] = lg;
  }
  __syncthreads();

  // softmax over the sources (every wave forms the weights it needs from the shared logits)
  float mx = -INFINITY;
  for (int s = 0; s < n_sources; ++s) mx = fmaxf(mx, s_logit[s]);
  float den = 0.f;
  for (int s = 0; s < n_sources; ++s) den += __expf(s_logit[s] - mx);
  const float inv_den = 1.f / den;

  // pass 2: sum_s round(w_s x_s) over this wave's sources (rows found in L2)
  float acc[NCH][8];
#pragma unroll
  for (int c = 0; c < NCH; ++c)
    for (int i = 0; i < 8; ++i) acc[c][i] = 0.f;
  for (int s = wave; s < n_sources; s += AR_WAVES) {
    const float w = round_to_t<T>(__expf(s_logit[s] - mx) * inv_den);
    float x[NCH][8];
    load_row(s, x);
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[c][i] += round_to_t<T>(x[c][i] * w);
  }
#pragma unroll
  for (int c = 0; c < NCH; ++c)
#pragma unroll
    for (int i = 0; i < 8; ++i) s_acc[wave][c * 8 + i][lane] = acc[c][i];
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (!on[c]) continue;
      float o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < AR_WAVES; ++w) v += s_acc[w][c * 8 + i][lane];
        o[i] = v;
      }
      row8<T>::store(out + (size_t)token * dim + 8 * (lane + 64 * c), o);
    }
  }
}

// The register-resident form (the release LM's bank: dim 1024, up to 64 sources): a workgroup of W waves per
// token (4 for a bf16 bank, 8 for fp32); wave w owns the sources w + W j (j < R), issues all their loads at
// once and holds the raw rows in registers for both passes (each row read from memory once). (A persistent
// form that loaded the next token's rows into a second register set while mixing the current one measured
// slower: the second set halves the resident workgroups.)
template <typename T>
struct raw8;  // 8 consecutive elements as loaded
template <>
struct raw8<bf16> {
  using type = uint4;
  __device__ __forceinline__ static type load(const bf16* p) { return *reinterpret_cast<const uint4*>(p); }
  __device__ __forceinline__ static void unpack(type w, float* f) {
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(u[i] << 16);
      f[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
    }
  }
};
template <>
struct raw8<float> {
  struct type {
    float4 a, b;
  };
  __device__ __forceinline__ static type load(const float* p) {
    return {*reinterpret_cast<const float4*>(p), *reinterpret_cast<const float4*>(p + 4)};
  }
  __device__ __forceinline__ static void unpack(type w, float* f) {
    f[0] = w.a.x; f[1] = w.a.y; f[2] = w.a.z; f[3] = w.a.w; f[4] = w.b.x; f[5] = w.b.y; f[6] = w.b.z; f[7] = w.b.w;
  }
};

template <typename T, int NCH, int R>
struct RowSet {
  typename raw8<T>::type x[R][NCH];
};

// The query as the passes use it: for bf16, each pair word split into (q_2i, 0) and (0, q_2i+1) words; for fp32
// the values.
template <typename T, int NCH>
struct QueryRegs {
  uint32_t lo[NCH][4], hi[NCH][4];
  float f[NCH][8];
};

// Every owned row of one token: the row pointers first (scalar loads, all in flight together), then the rows,
// unconditionally (a wave's slots past the last source re-read the last source's row and columns past dim
// re-read the row's last 8 columns; both are ignored), so that the compiler's wait counts stay exact.
template <typename T, int NCH, int R, int W>
__device__ __forceinline__ RowSet<T, NCH, R> load_rowset(const SourcePtrs& src, int n_sources, int dim,
                                                         long row_stride, int token, int wave, int lane) {
  RowSet<T, NCH, R> rs;
  const T* rows[R];
#pragma unroll
  for (int j = 0; j < R; ++j)
    rows[j] = reinterpret_cast<const T*>(src.p[min(wave + W * j, n_sources - 1)]) + (size_t)token * row_stride;
#pragma unroll
  for (int j = 0; j < R; ++j)
#pragma unroll
    for (int c = 0; c < NCH; ++c) rs.x[j][c] = raw8<T>::load(rows[j] + min(8 * (lane + 64 * c), dim - 8));
  return rs;
}

template <typename T, int NCH, int R, int W>
struct MixSm {
  // the waves' partial mixes, element (c, i) of lane l at [wave][8 c + i][l] (rows padded to 72 floats so that
  // the final sums' reads, 4 lanes x 4 element pairs, fall on 64 different banks)
  float acc[W][NCH * 8][72];
  float logit[AR_MAX_SOURCES];
};

// The cross-lane sums of R per-lane values at once: each v[j] becomes the sum over the wave's 64 lanes, as a
// wave-uniform value. Row sums by DPP; then the gfx950 permlane swaps, shared by 2 or 4 values: a 16-lane swap of
// a and b leaves a's row-pair sums in rows 0 and 2 and b's in rows 1 and 3, a 32-lane swap of two such results
// leaves four totals in rows 0-3, read with readlane. Each total is (s0 + s1) + (s2 + s3) of its row sums, the
// value wave_sum forms.
template <int R>
__device__ __forceinline__ void wave_sums(float (&v)[R]) {
#pragma unroll
  for (int j = 0; j < R; ++j) v[j] = group_sum<16>(v[j]);
  auto pair16 = [](float a, float b) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
  };
  auto pair32 = [](float a, float b) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
  };
  auto at = [](float x, int l) { return __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(x), l)); };
  int j = 0;
#pragma unroll
  for (; j + 4 <= R; j += 4) {
    const float t = pair32(pair16(v[j], v[j + 1]), pair16(v[j + 2], v[j + 3]));
    v[j] = at(t, 0);
    v[j + 1] = at(t, 16);
    v[j + 2] = at(t, 32);
    v[j + 3] = at(t, 48);
  }
  if constexpr (R % 4 >= 2) {
    const float ab = pair16(v[R / 4 * 4], v[R / 4 * 4 + 1]), t = pair32(ab, ab);
    v[R / 4 * 4] = at(t, 0);
    v[R / 4 * 4 + 1] = at(t, 16);
  }
  if constexpr (R % 2 == 1) {
    const float a = pair16(v[R - 1], v[R - 1]), t = pair32(a, a);
    v[R - 1] = at(t, 0);
  }
}

// One token's mix from its rows in registers. Two workgroup barriers: after the logits (before the softmax
// reads them) and after the partial mixes (before the final sums read them). FULL: dim == 512 NCH (every
// lane's pieces are columns of the row; no per-piece tests).
template <typename T, int NCH, int R, int W, bool FULL>
__device__ __forceinline__ void mix_token(const RowSet<T, NCH, R> xr, const QueryRegs<T, NCH> qr,
                                          MixSm<T, NCH, R, W>& sm, int n_sources, int dim, float eps, int token,
                                          int wave, int lane, T* __restrict__ out) {
  bool on[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) on[c] = FULL || 8 * (lane + 64 * c) < dim;
  const float inv_dim = 1.f / (float)dim;
  // pass 1: logit_s = sum round(round(x r) q), r = rsqrt(mean(x^2) + eps). Every owned slot is computed (a slot
  // past the last source holds that source's row again: finite values, never stored), so that the slots'
  // cross-lane sums run together.
  float ss[R], lg[R];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    ss[j] = 0.f;
    if constexpr (sizeof(T) == 2) {
      // bf16 bank: the same rounding points with the exact products and the fp32 sums on v_dot2c_f32_bf16
#pragma unroll
      for (int c = 0; c < NCH; ++c)
        if (on[c]) {
          const uint4 w = xr.x[j][c];
          ss[j] = dot2_bf16(w.x, w.x, dot2_bf16(w.y, w.y, dot2_bf16(w.z, w.z, dot2_bf16(w.w, w.w, ss[j]))));
        }
    } else {
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        float x[8];
        raw8<T>::unpack(xr.x[j][c], x);
#pragma unroll
        for (int i = 0; i < 8; ++i) ss[j] = fmaf(on[c] ? x[i] : 0.f, on[c] ? x[i] : 0.f, ss[j]);
      }
    }
  }
  wave_sums<R>(ss);
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const float r = rsqrtf(ss[j] * inv_dim + eps);
    lg[j] = 0.f;
    if constexpr (sizeof(T) == 2) {
      // per piece in stages (the keys, the 8 products, their packing, the sums), so that independent
      // instructions fill the wait states between a product and the conversion that reads it
#pragma unroll
      for (int c = 0; c < NCH; ++c)
        if (on[c]) {
          const uint4 w = xr.x[j][c];
          const uint32_t u[4] = {w.x, w.y, w.z, w.w};
          uint32_t k[4], pq[4];
#pragma unroll
          for (int i = 0; i < 4; ++i)
            k[i] = pack_bf16x2(__uint_as_float(u[i] << 16) * r, __uint_as_float(u[i] & 0xffff0000u) * r);
          products8(k, qr.lo[c], qr.hi[c], pq);
#pragma unroll
          for (int i = 0; i < 4; ++i) lg[j] = dot2_bf16(pq[i], BF16_ONES, lg[j]);
        }
    } else {
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        float x[8];
        raw8<T>::unpack(xr.x[j][c], x);
#pragma unroll
        for (int i = 0; i < 8; ++i) lg[j] += (on[c] ? x[i] : 0.f) * r * qr.f[c][i];
      }
    }
  }
  wave_sums<R>(lg);
#pragma unroll
  for (int j = 0; j < R; ++j)
    if (wave + W * j < n_sources && lane == 0) sm.logit[wave + W * j] = lg[j];
  __syncthreads();
  // softmax with one source per lane: e_s = exp(logit_s - max) in lane s, weight_s = e_s / sum e
  // (the cross-lane reductions run with every lane active)
  const float lg_l = lane < n_sources ? sm.logit[lane] : -INFINITY;
  const float mx = wave_max(lg_l);
  const float e_l = lane < n_sources ? __expf(lg_l - mx) : 0.f;
  const float inv_den = 1.f / wave_sum(e_l);
  // pass 2: sum_s round(w_s x_s) over this wave's sources
  float acc[NCH][8];
#pragma unroll
  for (int c = 0; c < NCH; ++c)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[c][i] = 0.f;
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int s = wave + W * j;
    if (s >= n_sources) break;
    // (s is wave-uniform: a lane read into a scalar register, no LDS round trip)
    const float w = round_to_t<T>(__uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(e_l), s)) * inv_den);
    if constexpr (sizeof(T) == 2) {
      // round(x w): exact products on (w, 0) / (0, w) words; the fp32 sums on (1, 0) / (0, 1) words
      const uint32_t wl = __float_as_uint(w) >> 16, wh = __float_as_uint(w) & 0xffff0000u;
      const uint32_t one_lo = bf16_one_lo();
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const uint4 xw = xr.x[j][c];
        const uint32_t u[4] = {xw.x, xw.y, xw.z, xw.w};
        const uint32_t wlo[4] = {wl, wl, wl, wl}, whi[4] = {wh, wh, wh, wh};
        uint32_t y[4];
        products8(u, wlo, whi, y);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[c][2 * i] = dot2_bf16(y[i], one_lo, acc[c][2 * i]);
          acc[c][2 * i + 1] = dot2_bf16(y[i], BF16_ONE_HI, acc[c][2 * i + 1]);
        }
      }
    } else {
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        float x[8];
        raw8<T>::unpack(xr.x[j][c], x);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[c][i] += x[i] * w;
      }
    }
  }
  // the waves' partial mixes through LDS; then every thread finishes two adjacent columns (a wave 128 of them)
#pragma unroll
  for (int c = 0; c < NCH; ++c)
#pragma unroll
    for (int i = 0; i < 8; ++i) sm.acc[wave][c * 8 + i][lane] = acc[c][i];
  __syncthreads();
  for (int pr = threadIdx.x; pr < NCH * 256; pr += 64 * W) {
    const int col = 2 * pr, c = col >> 9, l = (col & 511) >> 3, i = col & 7;
    if (col >= dim) break;
    float o0 = 0.f, o1 = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      o0 += sm.acc[w][c * 8 + i][l];
      o1 += sm.acc[w][c * 8 + i + 1][l];
    }
    if constexpr (sizeof(T) == 2)
      *reinterpret_cast<uint32_t*>(out + (size_t)token * dim + col) = pack_bf16x2(o0, o1);
    else
      *reinterpret_cast<float2*>(out + (size_t)token * dim + col) = make_float2(o0, o1);
  }
}

template <typename T, int NCH, int R, int W, bool FULL>
__global__ __launch_bounds__(64 * W) void attnres_reg_kernel(const SourcePtrs src, int n_sources, int tokens,
                                                             int dim, long row_stride, const T* __restrict__ query,
                                                             float eps, T* __restrict__ out, int n_cu, int per) {
  __shared__ MixSm<T, NCH, R, W> sm;
  const int t = cu_local_token(blockIdx.x, tokens, n_cu, per);
  if (t < 0) return;
  const int lane = threadIdx.x & 63, wave = wave_id();
  QueryRegs<T, NCH> qr;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const bool on = 8 * (lane + 64 * c) < dim;
    if constexpr (sizeof(T) == 2) {
      const uint4 w = on ? *reinterpret_cast<const uint4*>(query + 8 * (lane + 64 * c)) : make_uint4(0, 0, 0, 0);
      const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        qr.lo[c][i] = u[i] & 0xffffu;
        qr.hi[c][i] = u[i] & 0xffff0000u;
      }
    } else {
      if (on) row8<T>::load(query + 8 * (lane + 64 * c), qr.f[c]);
      else
        for (int i = 0; i < 8; ++i) qr.f[c][i] = 0.f;
    }
  }
  mix_token<T, NCH, R, W, FULL>(load_rowset<T, NCH, R, W>(src, n_sources, dim, row_stride, t, wave, lane), qr, sm,
                          n_sources, dim, eps, t, wave, lane, out);
}

template <typename T>
void launch_attnres(const SourcePtrs& p, int n_sources, int tokens, int dim, long row_stride, const void* query,
                    float eps, void* out, hipStream_t stream) {
  int dev = 0, n_cu = 256;  // the device's CUs, for the token mapping (cu_local_token)
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    n_cu = 256;
  n_cu = std::max(1, n_cu);
  const int per = tokens >= n_cu ? (tokens + n_cu - 1) / n_cu : 0;  // tokens per CU (0: one per workgroup)
  const int blocks = per > 0 ? n_cu * per : tokens;
  const int nch = (dim + 511) / 512;
  constexpr int W = sizeof(T) == 2 ? 4 : 8;  // waves per token of the register-resident form
  const int r = (n_sources + W - 1) / W;     // rows per wave
  const int rr = r <= 4 ? r : r <= 6 ? 6 : 8;
  if (nch <= 2 && nch * rr * (int)sizeof(T) * 8 <= 256) {  // raw rows held per lane: at most 256 bytes
    const bool full = dim == 512 * nch;
#define ZGDN_ARR_CASE(N, RR)                                                                                    \
  if (nch == N && rr == RR) {                                                                                   \
    if (full)                                                                                                   \
      hipLaunchKernelGGL((attnres_reg_kernel<T, N, RR, W, true>), dim3(blocks), dim3(64 * W), 0, stream, p,    \
                         n_sources, tokens, dim, row_stride, (const T*)query, eps, (T*)out, n_cu, per);        \
    else                                                                                                        \
      hipLaunchKernelGGL((attnres_reg_kernel<T, N, RR, W, false>), dim3(blocks), dim3(64 * W), 0, stream, p,   \
                         n_sources, tokens, dim, row_stride, (const T*)query, eps, (T*)out, n_cu, per);        \
    return;                                                                                                     \
  }
    ZGDN_ARR_CASE(1, 1) ZGDN_ARR_CASE(1, 2) ZGDN_ARR_CASE(1, 3) ZGDN_ARR_CASE(1, 4) ZGDN_ARR_CASE(1, 6)
    ZGDN_ARR_CASE(1, 8) ZGDN_ARR_CASE(2, 1) ZGDN_ARR_CASE(2, 2) ZGDN_ARR_CASE(2, 3) ZGDN_ARR_CASE(2, 4)
    ZGDN_ARR_CASE(2, 6) ZGDN_ARR_CASE(2, 8)
#undef ZGDN_ARR_CASE
  }
  dim3 grid(blocks), block(64 * AR_WAVES);
#define ZGDN_AR_CASE(N)                                                                                        \
  case N:                                                                                                      \
    hipLaunchKernelGGL((attnres_kernel<T, N>), grid, block, 0, stream, p, n_sources, dim, row_stride,         \
                       (const T*)query, eps, (T*)out, tokens, n_cu, per);                                      \
    break;
  switch (nch) {
    ZGDN_AR_CASE(1)
    ZGDN_AR_CASE(2)
    ZGDN_AR_CASE(3)
    ZGDN_AR_CASE(4)
  }
#undef ZGDN_AR_CASE
}

}  // namespace
}  // namespace zgdn

extern "C" int zgdn_attnres_route(const void* const* sources, int n_sources, int tokens, int dim, long row_stride,
                                  int dtype, const void* query, float eps, void* out, void* stream) {
  using namespace zgdn;
  const char* fn = "zgdn_attnres_route";
  if (!sources || !query || !out) return fail(ZGDN_EINVAL, "%s: null pointer", fn);
  if (n_sources < 1 || n_sources > AR_MAX_SOURCES)
    return fail(ZGDN_EUNSUPPORTED, "%s: %d sources (supported: 1..%d)", fn, n_sources, AR_MAX_SOURCES);
  if (tokens < 0 || dim < 8 || dim % 8 || dim > 2048)
    return fail(ZGDN_EUNSUPPORTED, "%s: tokens=%d dim=%d (dim a multiple of 8, <= 2048)", fn, tokens, dim);
  if (row_stride < dim || row_stride % 8)
    return fail(ZGDN_EINVAL, "%s: row stride %ld for dim %d (>= dim, a multiple of 8)", fn, row_stride, dim);
  if (dtype != ZGDN_F32 && dtype != ZGDN_BF16) return fail(ZGDN_EINVAL, "%s: dtype code %d", fn, dtype);
  SourcePtrs p{};
  for (int s = 0; s < n_sources; ++s) {
    if (!sources[s]) return fail(ZGDN_EINVAL, "%s: null source %d", fn, s);
    p.p[s] = sources[s];
  }
  if (tokens == 0) return check_launch(fn);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == ZGDN_F32)
    launch_attnres<float>(p, n_sources, tokens, dim, row_stride, query, eps, out, st);
  else
    launch_attnres<bf16>(p, n_sources, tokens, dim, row_stride, query, eps, out, st);
  return check_launch(fn);
}
