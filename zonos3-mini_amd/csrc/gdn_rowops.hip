// Row-local operators of the GDN layer: depthwise causal conv1d (+ SiLU) with a rolling history over packed
// sequences, q/k L2-norm, beta sigmoid and the gated RMSNorm of the output. All are HBM-streaming kernels:
// consecutive threads own consecutive channels / elements, so every global access is coalesced.
#include <type_traits>

#include "gdn_common.h"

namespace zgdn {
namespace {

constexpr int CONV_CH = 64;       // tokens per chunk of the chunk table
constexpr int CONV_TT = 8;        // tokens per conv workgroup (16 measured 14 % slower at 4096 x 1536)
constexpr int CONV_SPLIT = CONV_CH / CONV_TT;  // workgroups per chunk
constexpr int CONV_THREADS = 256;
constexpr int CONV_WMAX = 4;

template <typename T>
__device__ __forceinline__ float rnd(float x) {
  if constexpr (sizeof(T) == 2) return bf16_to_f32(f32_to_bf16(x));
  else return x;
}

// CPT consecutive channels as loaded / stored by one thread (one 4-byte word for two bf16, a float2 for two
// floats).
__device__ __forceinline__ float as_float(float x) { return x; }
__device__ __forceinline__ float as_float(bf16 x) { return bf16_to_f32(x.bits); }

template <typename T, int CPT>
struct chans;
// ``raw`` is the loaded word(s), converted to floats by ``unpack`` where the values are used (so issuing a
// load never waits for its data).
template <typename T>
struct chans<T, 1> {
  using raw = T;
  __device__ __forceinline__ static raw load(const T* p) { return *p; }
  __device__ __forceinline__ static void unpack(raw w, float* v) { v[0] = as_float(w); }
  __device__ __forceinline__ static void store(T* p, const float* v) { io<T>::store(p, v[0]); }
};
template <>
struct chans<bf16, 2> {
  using raw = uint32_t;
  __device__ __forceinline__ static raw load(const bf16* p) { return *reinterpret_cast<const uint32_t*>(p); }
  __device__ __forceinline__ static void unpack(raw w, float* v) {
    v[0] = __uint_as_float(w << 16);
    v[1] = __uint_as_float(w & 0xffff0000u);
  }
  __device__ __forceinline__ static void store(bf16* p, const float* v) {
    *reinterpret_cast<uint32_t*>(p) = pack_bf16x2(v[0], v[1]);
  }
};
template <>
struct chans<float, 2> {
  using raw = float2;
  __device__ __forceinline__ static raw load(const float* p) { return *reinterpret_cast<const float2*>(p); }
  __device__ __forceinline__ static void unpack(raw w, float* v) {
    v[0] = w.x;
    v[1] = w.y;
  }
  __device__ __forceinline__ static void store(float* p, const float* v) {
    *reinterpret_cast<float2*>(p) = make_float2(v[0], v[1]);
  }
};

// y[t, c] = act(sum_j w[c, j] * x_{t - W + 1 + j}[c] + bias[c]) over CONV_TT tokens of one chunk of one
// sequence (x rows x_ld elements apart, y rows dense), CPT channels per thread, with x_{<0} taken from the sequence's history (the last W-1 columns of
// its state row, oldest first); the first tile of a sequence also writes the new state row = the last SW raw
// inputs of [history | x]. The accumulation is fp32; like F.conv1d and F.silu on `T` tensors, the conv
// result is rounded to T before the activation and the activation after. A tile issues all its token loads
// before the arithmetic, so its latency is one load round trip rather than one per token.
template <typename T, int CPT, int WK>
__global__ __launch_bounds__(CONV_THREADS) void conv_kernel(
    const T* __restrict__ x, const T* __restrict__ w, const T* __restrict__ bias, const T* init, T* fin,
    T* __restrict__ y, const int32_t* __restrict__ cu, const int32_t* __restrict__ chunk_idx, int n_seqs,
    int n_chunks, int T_len, int D, long x_ld, int W_arg, int SW, int act) {
  const int W = WK > 0 ? WK : W_arg;  // WK: the width as a constant (the model's 4), 0: taken at run time
  const int c0 = (blockIdx.y * CONV_THREADS + threadIdx.x) * CPT;
  if (c0 >= D) return;
  int seq, j;
  const int tile = blockIdx.x / CONV_SPLIT, sub = blockIdx.x % CONV_SPLIT;
  if (cu != nullptr && (int)blockIdx.x >= n_chunks * CONV_SPLIT) {
    // trailing workgroups, one per sequence: empty packed sequences pass their state row through (zeros
    // without one)
    seq = blockIdx.x - n_chunks * CONV_SPLIT;
    int sb, se;
    seq_bounds(cu, seq, T_len, sb, se);
    if (fin == nullptr || se != sb) return;
    for (int k = 0; k < CPT; ++k) {
      T* frow = fin + ((size_t)seq * D + c0 + k) * SW;
      const T* hrow = init != nullptr ? init + ((size_t)seq * D + c0 + k) * SW : nullptr;
      for (int i = 0; i < SW; ++i) io<T>::store(frow + i, hrow != nullptr ? io<T>::load(hrow + i) : 0.f);
    }
    return;
  }
  if (cu != nullptr) {
    seq = chunk_idx[2 * tile];
    j = chunk_idx[2 * tile + 1];
    if (seq < 0 || seq >= n_seqs || j < 0) return;
  } else {
    const int nt = max(1, (T_len + CONV_CH - 1) / CONV_CH);
    seq = tile / nt;
    j = tile % nt;
  }
  int bos = seq * T_len, len = T_len;
  if (cu != nullptr) {
    int eos;
    seq_bounds(cu, seq, T_len, bos, eos);
    len = eos - bos;
  }
  const bool writes_state = fin != nullptr && j == 0 && sub == 0;
  if (len == 0) {  // an empty sequence (a batch of T = 0) passes its state row through
    if (writes_state)
      for (int k = 0; k < CPT; ++k) {
        T* frow = fin + ((size_t)seq * D + c0 + k) * SW;
        const T* hrow = init != nullptr ? init + ((size_t)seq * D + c0 + k) * SW : nullptr;
        for (int i = 0; i < SW; ++i) io<T>::store(frow + i, hrow != nullptr ? io<T>::load(hrow + i) : 0.f);
      }
    return;
  }
  if (j >= (len + CONV_CH - 1) / CONV_CH) return;  // a table row past the sequence's chunks
  const int t0 = j * CONV_CH + sub * CONV_TT;
  const int t1 = min(len, t0 + CONV_TT);
  if (t0 >= len) return;

  // Every load below is unconditional (indices clamped into the sequence / state row, a missing state row
  // replaced by x) and its value selected afterwards, so all of them issue back to back: a value written on
  // one side of a branch and loaded on the other would make the compiler wait for each load in turn.
  using C = chans<T, CPT>;
  const int last = len - 1;
  // Weights, bias, the tile's inputs and its history inside the sequence, all issued back to back with no
  // condition (indices clamped into the sequence). Only a sequence's first tile needs the old state row
  // (history before token 0) and the inputs of the new one; those loads come after, under conditions that
  // are false for every other tile. Raw words are converted when used.
  T wr[CPT][CONV_WMAX], br[CPT], hx[CPT][CONV_WMAX], hs[CPT][CONV_WMAX] = {}, nx[CPT][CONV_WMAX] = {},
      ns[CPT][CONV_WMAX] = {};
  typename C::raw xr[CONV_TT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int c = c0 + k;
#pragma unroll
    for (int i = 0; i < CONV_WMAX; ++i) wr[k][i] = w[(size_t)c * W + min(i, W - 1)];
    br[k] = (bias != nullptr ? bias : w)[bias != nullptr ? c : 0];
  }
#pragma unroll
  for (int i = 0; i < CONV_TT; ++i) xr[i] = C::load(x + ((size_t)(bos + min(t0 + i, last))) * x_ld + c0);
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const T* xc = x + (size_t)bos * x_ld + c0 + k;
#pragma unroll
    for (int i = 0; i < CONV_WMAX; ++i) hx[k][i] = xc[(size_t)min(max(t0 - (W - 1) + i, 0), last) * x_ld];
  }
  if (init != nullptr && (t0 < W - 1 || writes_state)) {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const T* hrow = init + ((size_t)seq * D + c0 + k) * SW;
#pragma unroll
      for (int i = 0; i < CONV_WMAX; ++i) {
        hs[k][i] = hrow[min(max(SW + t0 - (W - 1) + i, 0), SW - 1)];  // the input W-1-i steps before t0
        ns[k][i] = hrow[min(max(SW + len - SW + i, 0), SW - 1)];      // the new row's i-th input
      }
    }
  }
  if (writes_state) {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const T* xc = x + (size_t)bos * x_ld + c0 + k;
#pragma unroll
      for (int i = 0; i < CONV_WMAX; ++i) nx[k][i] = xc[(size_t)min(max(len - SW + i, 0), last) * x_ld];
    }
  }
  // values used (a missing state row reads as zeros)
  float wc[CPT][CONV_WMAX], hist[CPT][CONV_WMAX], nv[CPT][CONV_WMAX], bc[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    bc[k] = bias != nullptr ? as_float(br[k]) : 0.f;
#pragma unroll
    for (int i = 0; i < CONV_WMAX; ++i) {
      wc[k][i] = i < W ? as_float(wr[k][i]) : 0.f;
      const int th = t0 - (W - 1) + i, tn = len - SW + i;
      hist[k][i] = i >= W - 1 ? 0.f : th >= 0 ? as_float(hx[k][i]) : as_float(hs[k][i]);
      nv[k][i] = tn >= 0 ? as_float(nx[k][i]) : as_float(ns[k][i]);
    }
  }
  // full tiles (all but a sequence's last) run without a per-token guard
  auto run = [&](auto full) {
#pragma unroll
    for (int i = 0; i < CONV_TT; ++i) {
      if (!decltype(full)::value && t0 + i >= t1) continue;  // (not a break: the loop stays unrolled)
      float xv[CPT], out[CPT];
      C::unpack(xr[i], xv);
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        float acc = bc[k];
#pragma unroll
        for (int m = 0; m < CONV_WMAX - 1; ++m)
          if (m < W - 1) acc = fmaf(wc[k][m], hist[k][m], acc);
        out[k] = fmaf(wc[k][W - 1], xv[k], acc);
#pragma unroll
        for (int m = 0; m < CONV_WMAX - 2; ++m)
          if (m < W - 2) hist[k][m] = hist[k][m + 1];
        if (W >= 2) hist[k][W - 2] = xv[k];
      }
      // the conv rounded to T (two bf16 values with one conversion), then the activation; its result is rounded
      // to T by the store
      if constexpr (sizeof(T) == 2 && CPT == 2) {
        const uint32_t pk = pack_bf16x2(out[0], out[1]);
        out[0] = __uint_as_float(pk << 16);
        out[1] = __uint_as_float(pk & 0xffff0000u);
      } else {
#pragma unroll
        for (int k = 0; k < CPT; ++k) out[k] = rnd<T>(out[k]);
      }
      if (act) {
#pragma unroll
        for (int k = 0; k < CPT; ++k) out[k] = silu_fast(out[k]);
      }
      chans<T, CPT>::store(y + ((size_t)(bos + t0 + i)) * D + c0, out);
    }
  };
  if (t1 - t0 == CONV_TT)
    run(std::true_type{});
  else
    run(std::false_type{});
  // the tile holding the sequence start writes the new state row (it alone reads the old one, so the state
  // may be updated in place)
  if (writes_state) {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      T* frow = fin + ((size_t)seq * D + c0 + k) * SW;
#pragma unroll
      for (int i = 0; i < CONV_WMAX; ++i)
        if (i < SW) io<T>::store(frow + i, nv[k][i]);
    }
  }
}

// Rows of 128 (the head size): 16 lanes per row, each with 8 consecutive elements in one 16-byte access
// (two for fp32; element by element where some row is not 16-byte aligned, ALIGNED false, with the same
// arithmetic, so results do not depend on where the rows sit; every D = 128 call runs these kernels), and the row sum over the 16 lanes by DPP;
// four rows per wave.
template <typename T>
struct oct;
template <>
struct oct<bf16> {
  using raw = uint4;
  __device__ __forceinline__ static raw load(const bf16* p) { return *reinterpret_cast<const uint4*>(p); }
  __device__ __forceinline__ static raw load_unaligned(const bf16* p) {
    uint32_t u[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) u[i] = (uint32_t)p[2 * i].bits | ((uint32_t)p[2 * i + 1].bits << 16);
    return make_uint4(u[0], u[1], u[2], u[3]);
  }
  __device__ __forceinline__ static void unpack(const raw& w, float* v) {
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(u[i] << 16);
      v[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
    }
  }
  __device__ __forceinline__ static void store(bf16* p, const float* v) {
    *reinterpret_cast<uint4*>(p) = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                              pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
  }
  __device__ __forceinline__ static void store_unaligned(bf16* p, const float* v) {
#pragma unroll
    for (int i = 0; i < 8; ++i) io<bf16>::store(p + i, v[i]);
  }
};
template <>
struct oct<float> {
  struct raw {
    float4 a, b;
  };
  __device__ __forceinline__ static raw load(const float* p) {
    return {reinterpret_cast<const float4*>(p)[0], reinterpret_cast<const float4*>(p)[1]};
  }
  __device__ __forceinline__ static raw load_unaligned(const float* p) {
    return {make_float4(p[0], p[1], p[2], p[3]), make_float4(p[4], p[5], p[6], p[7])};
  }
  __device__ __forceinline__ static void unpack(const raw& w, float* v) {
    v[0] = w.a.x, v[1] = w.a.y, v[2] = w.a.z, v[3] = w.a.w;
    v[4] = w.b.x, v[5] = w.b.y, v[6] = w.b.z, v[7] = w.b.w;
  }
  __device__ __forceinline__ static void store(float* p, const float* v) {
    reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
  __device__ __forceinline__ static void store_unaligned(float* p, const float* v) {
#pragma unroll
    for (int i = 0; i < 8; ++i) p[i] = v[i];
  }
};
constexpr int R128_ROWS = 16;  // rows per 256-thread workgroup

// A whole 16-lane group exits together, so the DPP sums read active lanes only.
template <typename TI, typename TO, bool ALIGNED>
__global__ __launch_bounds__(256) void l2norm128_kernel(const TI* __restrict__ x, TO* __restrict__ y,
                                                        float* __restrict__ rstd, int rows, int x_group,
                                                        long x_ld, float eps) {
  const int row = blockIdx.x * R128_ROWS + (threadIdx.x >> 4), sub = threadIdx.x & 15;
  if (row >= rows) return;
  const TI* xr = x + (size_t)(row / x_group) * x_ld + (size_t)(row % x_group) * 128 + 8 * sub;
  float v[8];
  oct<TI>::unpack(ALIGNED ? oct<TI>::load(xr) : oct<TI>::load_unaligned(xr), v);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss = fmaf(v[i], v[i], ss);
  const float r = rsqrtf(group_sum<16>(ss) + eps);
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] *= r;
  TO* yr = y + (size_t)row * 128 + 8 * sub;
  if constexpr (ALIGNED) oct<TO>::store(yr, v);
  else oct<TO>::store_unaligned(yr, v);
  if (rstd != nullptr && sub == 0) rstd[row] = r;
}

template <typename T, bool ALIGNED>
__global__ __launch_bounds__(256) void gated_rmsnorm128_kernel(const T* __restrict__ x, const T* __restrict__ g,
                                                               const T* __restrict__ w, T* __restrict__ y,
                                                               float* __restrict__ rstd, int rows, int g_group,
                                                               long g_ld, float eps) {
  const int row = blockIdx.x * R128_ROWS + (threadIdx.x >> 4), sub = threadIdx.x & 15;
  if (row >= rows) return;
  const T* xp = x + (size_t)row * 128 + 8 * sub;
  const T* gp = g + (size_t)(row / g_group) * g_ld + (size_t)(row % g_group) * 128 + 8 * sub;
  const typename oct<T>::raw xr = ALIGNED ? oct<T>::load(xp) : oct<T>::load_unaligned(xp);
  const typename oct<T>::raw gr = ALIGNED ? oct<T>::load(gp) : oct<T>::load_unaligned(gp);
  const typename oct<T>::raw wr = ALIGNED ? oct<T>::load(w + 8 * sub) : oct<T>::load_unaligned(w + 8 * sub);
  float v[8], gv[8], wv[8];
  oct<T>::unpack(xr, v);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss = fmaf(v[i], v[i], ss);
  const float r = rsqrtf(group_sum<16>(ss) / 128.f + eps);
  oct<T>::unpack(gr, gv);
  oct<T>::unpack(wr, wv);
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = rnd<T>(v[i] * r * wv[i]) * silu(gv[i]);
  T* yr = y + (size_t)row * 128 + 8 * sub;
  if constexpr (ALIGNED) oct<T>::store(yr, v);
  else oct<T>::store_unaligned(yr, v);
  if (rstd != nullptr && sub == 0) rstd[row] = r;
}

// Whether rows of 128 at base p, ld elements apart, suit the 16-byte accesses of the 128-wide kernels.
__host__ inline bool rows128(const void* p, long ld, size_t esz) {
  return (uintptr_t)p % 16 == 0 && (ld * (long)esz) % 16 == 0;
}

// y = x * rsqrt(sum x^2 + eps) over rows of D <= 1024 elements; one wave per row. y is dense; row r of x
// starts at x + (r / x_group) * x_ld + (r % x_group) * D (a token's per-head rows inside a wider row).
template <typename TI, typename TO>
__global__ __launch_bounds__(256) void l2norm_kernel(const TI* __restrict__ x, TO* __restrict__ y,
                                                     float* __restrict__ rstd, int rows, int D, int x_group,
                                                     long x_ld, float eps) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const TI* xr = x + (size_t)(row / x_group) * x_ld + (size_t)(row % x_group) * D;
  float v[16];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int c = lane + 64 * i;
    v[i] = c < D ? io<TI>::load(xr + c) : 0.f;
    ss = fmaf(v[i], v[i], ss);
  }
  const float r = rsqrtf(wave_sum(ss) + eps);
  TO* yr = y + (size_t)row * D;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int c = lane + 64 * i;
    if (c < D) io<TO>::store(yr + c, v[i] * r);
  }
  if (rstd != nullptr && lane == 0) rstd[row] = r;
}

template <typename TI, typename TO>
__global__ __launch_bounds__(256) void sigmoid_kernel(const TI* __restrict__ x, TO* __restrict__ y, size_t n,
                                                      float scale) {
  const size_t i = blockIdx.x * (size_t)256 + threadIdx.x;
  if (i < n) io<TO>::store(y + i, sigmoid(io<TI>::load(x + i)) * scale);
}

// y = (rms_norm(x) * w).to(T) * silu(g), product in fp32, cast to T; one wave per row of D <= 1024. x and y
// are dense; row r's gate starts at g + (r / g_group) * g_ld + (r % g_group) * D (per-head rows of a token's
// gate, read in place from a wider row).
template <typename T>
__global__ __launch_bounds__(256) void gated_rmsnorm_kernel(const T* __restrict__ x, const T* __restrict__ g,
                                                            const T* __restrict__ w, T* __restrict__ y,
                                                            float* __restrict__ rstd, int rows, int D, int g_group,
                                                            long g_ld, float eps) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const T* xr = x + (size_t)row * D;
  float v[16];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int c = lane + 64 * i;
    v[i] = c < D ? io<T>::load(xr + c) : 0.f;
    ss = fmaf(v[i], v[i], ss);
  }
  const float r = rsqrtf(wave_sum(ss) / (float)D + eps);
  const T* gr = g + (size_t)(row / g_group) * g_ld + (size_t)(row % g_group) * D;
  T* yr = y + (size_t)row * D;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int c = lane + 64 * i;
    if (c < D) io<T>::store(yr + c, rnd<T>(v[i] * r * io<T>::load(w + c)) * silu(io<T>::load(gr + c)));
  }
  if (rstd != nullptr && lane == 0) rstd[row] = r;
}

}  // namespace
}  // namespace zgdn

extern "C" int zgdn_causal_conv1d_fwd(const void* x, const void* weight, const void* bias, int dtype,
                                      const void* initial_state, void* final_state, int state_width, void* y,
                                      const int32_t* cu_seqlens, const int32_t* chunk_indices, int n_seqs,
                                      int n_chunks, int B, int T, int D, int W, int activation, long x_ld,
                                      void* stream) {
  using namespace zgdn;
  const char* fn = "zgdn_causal_conv1d_fwd";
  if (!x || !weight || !y) return fail(ZGDN_EINVAL, "%s: null pointer", fn);
  if (x_ld < D) return fail(ZGDN_EINVAL, "%s: x row stride %ld < D=%d", fn, x_ld, D);
  if (W < 1 || W > CONV_WMAX) return fail(ZGDN_EUNSUPPORTED, "%s: width %d (supported: 1..4)", fn, W);
  if (state_width < W - 1 || state_width > CONV_WMAX)
    return fail(ZGDN_EINVAL, "%s: state width %d for conv width %d (need W-1 .. 4)", fn, state_width, W);
  if (B < 1 || T < 0 || D < 1) return fail(ZGDN_EINVAL, "%s: bad sizes B=%d T=%d D=%d", fn, B, T, D);
  if (dtype != ZGDN_F32 && dtype != ZGDN_BF16) return fail(ZGDN_EINVAL, "%s: dtype code %d", fn, dtype);
  int grid_x;
  if (cu_seqlens != nullptr) {
    if (B != 1 || chunk_indices == nullptr || n_seqs < 1 || n_chunks < 0)
      return fail(ZGDN_EINVAL, "%s: packed sequences need B == 1, chunk_indices and n_seqs >= 1", fn);
    grid_x = n_chunks * CONV_SPLIT + n_seqs;  // + one workgroup column per sequence for empty ones
  } else {
    n_seqs = B;
    grid_x = B * ((T + CONV_CH - 1) / CONV_CH) * CONV_SPLIT;
    if (T == 0) grid_x = B * CONV_SPLIT;  // empty sequences still pass their state through
  }
  if (grid_x == 0) return check_launch(fn);
  hipStream_t s = (hipStream_t)stream;
  auto go = [&](auto* tag, auto cpt) {
    using TT = std::remove_pointer_t<decltype(tag)>;
    constexpr int CPT = decltype(cpt)::value;
    const int per_wg = CONV_THREADS * CPT;
    dim3 grid(grid_x, (D + per_wg - 1) / per_wg);
    auto kernel = W == 4 ? conv_kernel<TT, CPT, 4> : conv_kernel<TT, CPT, 0>;
    hipLaunchKernelGGL(kernel, grid, dim3(CONV_THREADS), 0, s, (const TT*)x, (const TT*)weight, (const TT*)bias,
                       (const TT*)initial_state, (TT*)final_state, (TT*)y, cu_seqlens, chunk_indices, n_seqs,
                       n_chunks, T, D, x_ld, W, state_width, activation);
  };
  using One = std::integral_constant<int, 1>;
  using Two = std::integral_constant<int, 2>;
  // two channels per thread where every pair of x and y stays 4- or 8-byte aligned (four bf16 channels a thread,
  // 8-byte accesses in 128-thread workgroups, measured 13 % slower at 4096 x 1536: more registers, fewer waves)
  const size_t esz = dtype == ZGDN_F32 ? 4 : 2;
  const bool pairs = D % 2 == 0 && x_ld % 2 == 0 && (uintptr_t)x % (2 * esz) == 0 && (uintptr_t)y % (2 * esz) == 0;
  if (dtype == ZGDN_F32) {
    if (pairs) go((float*)nullptr, Two{});
    else go((float*)nullptr, One{});
  } else {
    if (pairs) go((bf16*)nullptr, Two{});
    else go((bf16*)nullptr, One{});
  }
  return check_launch(fn);
}

extern "C" int zgdn_l2norm_fwd(const void* x, int x_dtype, void* y, int y_dtype, float* rstd, int rows, int D,
                               int x_group, long x_ld, float eps, void* stream) {
  using namespace zgdn;
  const char* fn = "zgdn_l2norm_fwd";
  if (!x || !y) return fail(ZGDN_EINVAL, "%s: null pointer", fn);
  if (rows < 0 || D < 1 || D > 1024) return fail(ZGDN_EUNSUPPORTED, "%s: rows=%d D=%d (D <= 1024)", fn, rows, D);
  if (x_group < 1 || x_ld < (long)x_group * D)
    return fail(ZGDN_EINVAL, "%s: x rows: group %d, stride %ld (need group >= 1, stride >= group * D)", fn,
                x_group, x_ld);
  for (int dt : {x_dtype, y_dtype})
    if (dt != ZGDN_F32 && dt != ZGDN_BF16) return fail(ZGDN_EINVAL, "%s: dtype code %d", fn, dt);
  if (rows == 0) return check_launch(fn);
  hipStream_t s = (hipStream_t)stream;
  if (D == 128) {
    const bool al = rows128(x, x_ld, x_dtype == ZGDN_F32 ? 4 : 2) && rows128(y, 128, y_dtype == ZGDN_F32 ? 4 : 2);
    dim3 grid((rows + R128_ROWS - 1) / R128_ROWS), block(256);
    auto go = [&](auto* ti, auto* to) {
      using TI = std::remove_const_t<std::remove_pointer_t<decltype(ti)>>;
      using TO = std::remove_pointer_t<decltype(to)>;
      auto kernel = al ? l2norm128_kernel<TI, TO, true> : l2norm128_kernel<TI, TO, false>;
      hipLaunchKernelGGL(kernel, grid, block, 0, s, (const TI*)x, (TO*)y, rstd, rows, x_group, x_ld, eps);
    };
    if (x_dtype == ZGDN_F32 && y_dtype == ZGDN_F32) go((float*)nullptr, (float*)nullptr);
    else if (x_dtype == ZGDN_F32) go((float*)nullptr, (bf16*)nullptr);
    else if (y_dtype == ZGDN_F32) go((bf16*)nullptr, (float*)nullptr);
    else go((bf16*)nullptr, (bf16*)nullptr);
    return check_launch(fn);
  }
  dim3 grid((rows + 3) / 4), block(256);
  if (x_dtype == ZGDN_F32 && y_dtype == ZGDN_F32)
    hipLaunchKernelGGL((l2norm_kernel<float, float>), grid, block, 0, s, (const float*)x, (float*)y, rstd, rows, D, x_group, x_ld, eps);
  else if (x_dtype == ZGDN_F32)
    hipLaunchKernelGGL((l2norm_kernel<float, bf16>), grid, block, 0, s, (const float*)x, (bf16*)y, rstd, rows, D, x_group, x_ld, eps);
  else if (y_dtype == ZGDN_F32)
    hipLaunchKernelGGL((l2norm_kernel<bf16, float>), grid, block, 0, s, (const bf16*)x, (float*)y, rstd, rows, D, x_group, x_ld, eps);
  else
    hipLaunchKernelGGL((l2norm_kernel<bf16, bf16>), grid, block, 0, s, (const bf16*)x, (bf16*)y, rstd, rows, D, x_group, x_ld, eps);
  return check_launch(fn);
}

extern "C" int zgdn_sigmoid_fwd(const void* x, int x_dtype, void* y, int y_dtype, size_t n, float scale,
                                void* stream) {
  using namespace zgdn;
  const char* fn = "zgdn_sigmoid_fwd";
  if (!x || !y) return fail(ZGDN_EINVAL, "%s: null pointer", fn);
  for (int dt : {x_dtype, y_dtype})
    if (dt != ZGDN_F32 && dt != ZGDN_BF16) return fail(ZGDN_EINVAL, "%s: dtype code %d", fn, dt);
  if (n == 0) return check_launch(fn);
  dim3 grid((unsigned)((n + 255) / 256)), block(256);
  hipStream_t s = (hipStream_t)stream;
  if (x_dtype == ZGDN_F32 && y_dtype == ZGDN_F32)
    hipLaunchKernelGGL((sigmoid_kernel<float, float>), grid, block, 0, s, (const float*)x, (float*)y, n, scale);
  else if (x_dtype == ZGDN_F32)
    hipLaunchKernelGGL((sigmoid_kernel<float, bf16>), grid, block, 0, s, (const float*)x, (bf16*)y, n, scale);
  else if (y_dtype == ZGDN_F32)
    hipLaunchKernelGGL((sigmoid_kernel<bf16, float>), grid, block, 0, s, (const bf16*)x, (float*)y, n, scale);
  else
    hipLaunchKernelGGL((sigmoid_kernel<bf16, bf16>), grid, block, 0, s, (const bf16*)x, (bf16*)y, n, scale);
  return check_launch(fn);
}

extern "C" int zgdn_gated_rmsnorm_fwd(const void* x, const void* g, const void* weight, int dtype, void* y,
                                      float* rstd, int rows, int D, int g_group, long g_ld, float eps,
                                      void* stream) {
  using namespace zgdn;
  const char* fn = "zgdn_gated_rmsnorm_fwd";
  if (!x || !g || !weight || !y) return fail(ZGDN_EINVAL, "%s: null pointer", fn);
  if (g_group < 1 || g_ld < (long)g_group * D)
    return fail(ZGDN_EINVAL, "%s: gate rows: group %d, stride %ld (need group >= 1, stride >= group * D)", fn,
                g_group, g_ld);
  if (rows < 0 || D < 1 || D > 1024) return fail(ZGDN_EUNSUPPORTED, "%s: rows=%d D=%d (D <= 1024)", fn, rows, D);
  if (dtype != ZGDN_F32 && dtype != ZGDN_BF16) return fail(ZGDN_EINVAL, "%s: dtype code %d", fn, dtype);
  if (rows == 0) return check_launch(fn);
  hipStream_t s = (hipStream_t)stream;
  const size_t esz = dtype == ZGDN_F32 ? 4 : 2;
  if (D == 128) {
    const bool al = rows128(x, 128, esz) && rows128(g, g_ld, esz) && rows128(weight, 0, esz) && rows128(y, 128, esz);
    dim3 grid((rows + R128_ROWS - 1) / R128_ROWS), block(256);
    auto go = [&](auto* tag) {
      using T = std::remove_pointer_t<decltype(tag)>;
      auto kernel = al ? gated_rmsnorm128_kernel<T, true> : gated_rmsnorm128_kernel<T, false>;
      hipLaunchKernelGGL(kernel, grid, block, 0, s, (const T*)x, (const T*)g, (const T*)weight, (T*)y, rstd, rows,
                         g_group, g_ld, eps);
    };
    if (dtype == ZGDN_F32) go((float*)nullptr);
    else go((bf16*)nullptr);
    return check_launch(fn);
  }
  dim3 grid((rows + 3) / 4), block(256);
  if (dtype == ZGDN_F32)
    hipLaunchKernelGGL(gated_rmsnorm_kernel<float>, grid, block, 0, s, (const float*)x, (const float*)g,
                       (const float*)weight, (float*)y, rstd, rows, D, g_group, g_ld, eps);
  else
    hipLaunchKernelGGL(gated_rmsnorm_kernel<bf16>, grid, block, 0, s, (const bf16*)x, (const bf16*)g,
                       (const bf16*)weight, (bf16*)y, rstd, rows, D, g_group, g_ld, eps);
  return check_launch(fn);
}
