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

// NCH: 8-element pieces per lane (dim <= 512 NCH); columns past dim are masked.
template <typename T, int NCH>
__global__ __launch_bounds__(64 * AR_WAVES) void attnres_kernel(const SourcePtrs src, int n_sources, int dim,
                                                                  long row_stride, const T* __restrict__ query,
                                                                  float eps, T* __restrict__ out) {
  __shared__ float s_acc[AR_WAVES][NCH * 8][64];
  __shared__ float s_logit[AR_MAX_SOURCES];
  const int token = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
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

// The register-resident form (the release LM's bank: dim 1024, up to 64 sources): AR_RWAVES waves per token,
// wave w owns sources w + AR_RWAVES j (j < R) and issues all their loads at once, keeping the raw rows in
// registers for both passes (each row read from memory once, no second read). Same arithmetic as above.
constexpr int AR_RWAVES = 8;

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
__global__ __launch_bounds__(64 * AR_RWAVES) void attnres_reg_kernel(const SourcePtrs src, int n_sources, int dim,
                                                                       long row_stride, const T* __restrict__ query,
                                                                       float eps, T* __restrict__ out) {
  __shared__ float s_acc[AR_RWAVES / 2][NCH * 8][64];
  __shared__ float s_logit[AR_MAX_SOURCES];
  const int token = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  bool on[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) on[c] = 8 * (lane + 64 * c) < dim;
  // every owned row's loads first (a source past n_sources or a column past dim is not read)
  typename raw8<T>::type xr[R][NCH];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int s = wave + AR_RWAVES * j;
    const T* row = reinterpret_cast<const T*>(src.p[min(s, n_sources - 1)]) + (size_t)token * row_stride;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      if (s < n_sources && on[c]) xr[j][c] = raw8<T>::load(row + 8 * (lane + 64 * c));
  }
  float q[NCH][8];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (on[c]) row8<T>::load(query + 8 * (lane + 64 * c), q[c]);
    else
      for (int i = 0; i < 8; ++i) q[c][i] = 0.f;
  }
  const float inv_dim = 1.f / (float)dim;
  // pass 1: logits
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int s = wave + AR_RWAVES * j;
    if (s >= n_sources) break;
    float x[NCH][8], ss = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (on[c]) raw8<T>::unpack(xr[j][c], x[c]);
      else
        for (int i = 0; i < 8; ++i) x[c][i] = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = fmaf(x[c][i], x[c][i], ss);
    }
    const float r = rsqrtf(wave_sum(ss) * inv_dim + eps);
    float lg = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        float k0 = x[c][i] * r, k1 = x[c][i + 1] * r;
        round2_t<T>(k0, k1);
        float p0 = k0 * q[c][i], p1 = k1 * q[c][i + 1];
        round2_t<T>(p0, p1);
        lg += p0;
        lg += p1;
      }
    lg = wave_sum(lg);
    if (lane == 0) s_logit[s] = lg;
  }
  __syncthreads();
  float mx = -INFINITY;
  for (int s = 0; s < n_sources; ++s) mx = fmaxf(mx, s_logit[s]);
  float den = 0.f;
  for (int s = 0; s < n_sources; ++s) den += __expf(s_logit[s] - mx);
  const float inv_den = 1.f / den;
  // pass 2 from the registers
  float acc[NCH][8];
#pragma unroll
  for (int c = 0; c < NCH; ++c)
    for (int i = 0; i < 8; ++i) acc[c][i] = 0.f;
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int s = wave + AR_RWAVES * j;
    if (s >= n_sources) break;
    const float w = round_to_t<T>(__expf(s_logit[s] - mx) * inv_den);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (!on[c]) continue;
      float x[8];
      raw8<T>::unpack(xr[j][c], x);
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        float y0 = x[i] * w, y1 = x[i + 1] * w;
        round2_t<T>(y0, y1);
        acc[c][i] += y0;
        acc[c][i + 1] += y1;
      }
    }
  }
  // waves 4-7 hand their sums to waves 0-3, each of which adds its partner's; wave 0 adds the four results
  if (wave >= AR_RWAVES / 2) {
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int i = 0; i < 8; ++i) s_acc[wave - AR_RWAVES / 2][c * 8 + i][lane] = acc[c][i];
  }
  __syncthreads();
  if (wave < AR_RWAVES / 2) {
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int i = 0; i < 8; ++i) s_acc[wave][c * 8 + i][lane] += acc[c][i];
  }
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
        for (int w = 0; w < AR_RWAVES / 2; ++w) v += s_acc[w][c * 8 + i][lane];
        o[i] = v;
      }
      row8<T>::store(out + (size_t)token * dim + 8 * (lane + 64 * c), o);
    }
  }
}

template <typename T>
void launch_attnres(const SourcePtrs& p, int n_sources, int tokens, int dim, long row_stride, const void* query,
                    float eps, void* out, hipStream_t stream) {
  const int nch = (dim + 511) / 512;
  const int r = (n_sources + AR_RWAVES - 1) / AR_RWAVES;  // rows per wave of the register-resident form
  const int rr = r <= 1 ? 1 : r <= 2 ? 2 : r <= 4 ? 4 : 8;
  if (nch <= 2 && nch * rr * (int)sizeof(T) * 8 <= 256) {  // raw rows held per lane: at most 256 bytes
#define ZGDN_ARR_CASE(N, RR)                                                                                    \
  if (nch == N && rr == RR) {                                                                                   \
    hipLaunchKernelGGL((attnres_reg_kernel<T, N, RR>), dim3(tokens), dim3(64 * AR_RWAVES), 0, stream, p,       \
                       n_sources, dim, row_stride, (const T*)query, eps, (T*)out);                             \
    return;                                                                                                     \
  }
    ZGDN_ARR_CASE(1, 1) ZGDN_ARR_CASE(1, 2) ZGDN_ARR_CASE(1, 4) ZGDN_ARR_CASE(1, 8)
    ZGDN_ARR_CASE(2, 1) ZGDN_ARR_CASE(2, 2) ZGDN_ARR_CASE(2, 4) ZGDN_ARR_CASE(2, 8)
#undef ZGDN_ARR_CASE
  }
  dim3 grid(tokens), block(64 * AR_WAVES);
#define ZGDN_AR_CASE(N)                                                                                        \
  case N:                                                                                                      \
    hipLaunchKernelGGL((attnres_kernel<T, N>), grid, block, 0, stream, p, n_sources, dim, row_stride,         \
                       (const T*)query, eps, (T*)out);                                                         \
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
