// Row-local operators of the GDN layer: depthwise causal conv1d (+ SiLU) with a rolling history over packed
// sequences, q/k L2-norm, beta sigmoid and the gated RMSNorm of the output. All are HBM-streaming kernels:
// consecutive threads own consecutive channels / elements, so every global access is coalesced.
#include "gdn_common.h"

namespace zgdn {
namespace {

constexpr int CONV_CH = 64;       // tokens per conv workgroup (the chunk length of the chunk table)
constexpr int CONV_THREADS = 256;
constexpr int CONV_WMAX = 4;

template <typename T>
__device__ __forceinline__ float rnd(float x) {
  if constexpr (sizeof(T) == 2) return bf16_to_f32(f32_to_bf16(x));
  else return x;
}

// y[t, c] = act(sum_j w[c, j] * x_{t - W + 1 + j}[c] + bias[c]) over the tokens of one chunk of one sequence,
// with x_{<0} taken from the sequence's history (the last W-1 columns of its state row, oldest first) and
// the new state row = the last SW raw inputs of [history | x]. The accumulation is fp32; like F.conv1d and
// F.silu on `T` tensors, the conv result is rounded to T before the activation and the activation after.
template <typename T>
__global__ __launch_bounds__(CONV_THREADS) void conv_kernel(
    const T* __restrict__ x, const T* __restrict__ w, const T* __restrict__ bias, const T* init, T* fin,
    T* __restrict__ y, const int32_t* __restrict__ cu, const int32_t* __restrict__ chunk_idx, int n_seqs,
    int n_chunks, int T_len, int D, int W, int SW, int act) {
  const int c = blockIdx.y * CONV_THREADS + threadIdx.x;
  if (c >= D) return;
  int seq, j;
  if (cu != nullptr && (int)blockIdx.x >= n_chunks) {
    // trailing workgroups: empty packed sequences pass their state row through (zeros without one)
    seq = blockIdx.x - n_chunks;
    if (fin == nullptr || cu[seq + 1] != cu[seq]) return;
    T* frow = fin + ((size_t)seq * D + c) * SW;
    const T* hrow = init != nullptr ? init + ((size_t)seq * D + c) * SW : nullptr;
    for (int i = 0; i < SW; ++i) io<T>::store(frow + i, hrow != nullptr ? io<T>::load(hrow + i) : 0.f);
    return;
  }
  if (cu != nullptr) {
    seq = chunk_idx[2 * blockIdx.x];
    j = chunk_idx[2 * blockIdx.x + 1];
    if (seq < 0 || seq >= n_seqs || j < 0) return;
  } else {
    const int nt = max(1, (T_len + CONV_CH - 1) / CONV_CH);
    seq = blockIdx.x / nt;
    j = blockIdx.x % nt;
  }
  const int bos = cu != nullptr ? cu[seq] : seq * T_len;
  const int len = cu != nullptr ? cu[seq + 1] - bos : T_len;
  const int t0 = j * CONV_CH;
  const int t1 = min(len, t0 + CONV_CH);
  if (t0 >= len && len > 0) return;

  float wc[CONV_WMAX], hist[CONV_WMAX];
#pragma unroll
  for (int i = 0; i < CONV_WMAX; ++i) wc[i] = i < W ? io<T>::load(w + (size_t)c * W + i) : 0.f;
  const float bc = bias != nullptr ? io<T>::load(bias + c) : 0.f;
  const T* hrow = init != nullptr ? init + ((size_t)seq * D + c) * SW : nullptr;
  // hist[i], i < W-1: the raw input W-1-i steps before token t0
#pragma unroll
  for (int i = 0; i < CONV_WMAX - 1; ++i) {
    float hv = 0.f;
    if (i < W - 1) {
      const int tt = t0 - (W - 1) + i;  // position within the sequence
      if (tt >= 0) hv = io<T>::load(x + ((size_t)(bos + tt)) * D + c);
      else if (hrow != nullptr) hv = io<T>::load(hrow + SW + tt);  // SW + tt >= SW - (W - 1) >= 0
    }
    hist[i] = hv;
  }
  for (int t = t0; t < t1; ++t) {
    const float xv = io<T>::load(x + ((size_t)(bos + t)) * D + c);
    float acc = bc;
#pragma unroll
    for (int i = 0; i < CONV_WMAX - 1; ++i)
      if (i < W - 1) acc = fmaf(wc[i], hist[i], acc);
    acc = fmaf(wc[W - 1], xv, acc);
    float out = rnd<T>(acc);
    if (act) out = rnd<T>(silu(out));
    io<T>::store(y + ((size_t)(bos + t)) * D + c, out);
#pragma unroll
    for (int i = 0; i < CONV_WMAX - 2; ++i)
      if (i < W - 2) hist[i] = hist[i + 1];
    if (W >= 2) hist[W - 2] = xv;
  }
  // the chunk holding the sequence start also writes the new state row (it alone reads the old one, so the
  // state may be updated in place): the last SW raw inputs of [history | x], oldest first
  if (fin != nullptr && j == 0) {
    T* frow = fin + ((size_t)seq * D + c) * SW;
    float nv[CONV_WMAX];
#pragma unroll
    for (int i = 0; i < CONV_WMAX; ++i) {
      nv[i] = 0.f;
      if (i < SW) {
        const int tt = len - SW + i;  // position within the sequence (negative: from the old history)
        if (tt >= 0) nv[i] = io<T>::load(x + ((size_t)(bos + tt)) * D + c);
        else if (hrow != nullptr) nv[i] = io<T>::load(hrow + SW + tt);
      }
    }
#pragma unroll
    for (int i = 0; i < CONV_WMAX; ++i)
      if (i < SW) io<T>::store(frow + i, nv[i]);
  }
}

// y = x * rsqrt(sum x^2 + eps) over rows of D <= 1024 elements; one wave per row.
template <typename TI, typename TO>
__global__ __launch_bounds__(256) void l2norm_kernel(const TI* __restrict__ x, TO* __restrict__ y,
                                                     float* __restrict__ rstd, int rows, int D, float eps) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const TI* xr = x + (size_t)row * D;
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

// y = (rms_norm(x) * w).to(T) * silu(g), product in fp32, cast to T; one wave per row of D <= 1024.
template <typename T>
__global__ __launch_bounds__(256) void gated_rmsnorm_kernel(const T* __restrict__ x, const T* __restrict__ g,
                                                            const T* __restrict__ w, T* __restrict__ y,
                                                            float* __restrict__ rstd, int rows, int D, float eps) {
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
  const T* gr = g + (size_t)row * D;
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
                                      int n_chunks, int B, int T, int D, int W, int activation, void* stream) {
  using namespace zgdn;
  const char* fn = "zgdn_causal_conv1d_fwd";
  if (!x || !weight || !y) return fail(ZGDN_EINVAL, "%s: null pointer", fn);
  if (W < 1 || W > CONV_WMAX) return fail(ZGDN_EUNSUPPORTED, "%s: width %d (supported: 1..4)", fn, W);
  if (state_width < W - 1 || state_width > CONV_WMAX)
    return fail(ZGDN_EINVAL, "%s: state width %d for conv width %d (need W-1 .. 4)", fn, state_width, W);
  if (B < 1 || T < 0 || D < 1) return fail(ZGDN_EINVAL, "%s: bad sizes B=%d T=%d D=%d", fn, B, T, D);
  if (dtype != ZGDN_F32 && dtype != ZGDN_BF16) return fail(ZGDN_EINVAL, "%s: dtype code %d", fn, dtype);
  int grid_x;
  if (cu_seqlens != nullptr) {
    if (B != 1 || chunk_indices == nullptr || n_seqs < 1 || n_chunks < 0)
      return fail(ZGDN_EINVAL, "%s: packed sequences need B == 1, chunk_indices and n_seqs >= 1", fn);
    grid_x = n_chunks + n_seqs;  // + one workgroup column per sequence for empty ones
  } else {
    n_seqs = B;
    grid_x = B * ((T + CONV_CH - 1) / CONV_CH);
    if (T == 0) grid_x = B;  // empty sequences still pass their state through
  }
  if (grid_x == 0) return check_launch(fn);
  dim3 grid(grid_x, (D + CONV_THREADS - 1) / CONV_THREADS);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ZGDN_F32)
    hipLaunchKernelGGL(conv_kernel<float>, grid, dim3(CONV_THREADS), 0, s, (const float*)x, (const float*)weight,
                       (const float*)bias, (const float*)initial_state, (float*)final_state, (float*)y, cu_seqlens,
                       chunk_indices, n_seqs, n_chunks, T, D, W, state_width, activation);
  else
    hipLaunchKernelGGL(conv_kernel<bf16>, grid, dim3(CONV_THREADS), 0, s, (const bf16*)x, (const bf16*)weight,
                       (const bf16*)bias, (const bf16*)initial_state, (bf16*)final_state, (bf16*)y, cu_seqlens,
                       chunk_indices, n_seqs, n_chunks, T, D, W, state_width, activation);
  return check_launch(fn);
}

extern "C" int zgdn_l2norm_fwd(const void* x, int x_dtype, void* y, int y_dtype, float* rstd, int rows, int D,
                               float eps, void* stream) {
  using namespace zgdn;
  const char* fn = "zgdn_l2norm_fwd";
  if (!x || !y) return fail(ZGDN_EINVAL, "%s: null pointer", fn);
  if (rows < 0 || D < 1 || D > 1024) return fail(ZGDN_EUNSUPPORTED, "%s: rows=%d D=%d (D <= 1024)", fn, rows, D);
  for (int dt : {x_dtype, y_dtype})
    if (dt != ZGDN_F32 && dt != ZGDN_BF16) return fail(ZGDN_EINVAL, "%s: dtype code %d", fn, dt);
  if (rows == 0) return check_launch(fn);
  dim3 grid((rows + 3) / 4), block(256);
  hipStream_t s = (hipStream_t)stream;
  if (x_dtype == ZGDN_F32 && y_dtype == ZGDN_F32)
    hipLaunchKernelGGL((l2norm_kernel<float, float>), grid, block, 0, s, (const float*)x, (float*)y, rstd, rows, D, eps);
  else if (x_dtype == ZGDN_F32)
    hipLaunchKernelGGL((l2norm_kernel<float, bf16>), grid, block, 0, s, (const float*)x, (bf16*)y, rstd, rows, D, eps);
  else if (y_dtype == ZGDN_F32)
    hipLaunchKernelGGL((l2norm_kernel<bf16, float>), grid, block, 0, s, (const bf16*)x, (float*)y, rstd, rows, D, eps);
  else
    hipLaunchKernelGGL((l2norm_kernel<bf16, bf16>), grid, block, 0, s, (const bf16*)x, (bf16*)y, rstd, rows, D, eps);
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
                                      float* rstd, int rows, int D, float eps, void* stream) {
  using namespace zgdn;
  const char* fn = "zgdn_gated_rmsnorm_fwd";
  if (!x || !g || !weight || !y) return fail(ZGDN_EINVAL, "%s: null pointer", fn);
  if (rows < 0 || D < 1 || D > 1024) return fail(ZGDN_EUNSUPPORTED, "%s: rows=%d D=%d (D <= 1024)", fn, rows, D);
  if (dtype != ZGDN_F32 && dtype != ZGDN_BF16) return fail(ZGDN_EINVAL, "%s: dtype code %d", fn, dtype);
  if (rows == 0) return check_launch(fn);
  dim3 grid((rows + 3) / 4), block(256);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ZGDN_F32)
    hipLaunchKernelGGL(gated_rmsnorm_kernel<float>, grid, block, 0, s, (const float*)x, (const float*)g,
                       (const float*)weight, (float*)y, rstd, rows, D, eps);
  else
    hipLaunchKernelGGL(gated_rmsnorm_kernel<bf16>, grid, block, 0, s, (const bf16*)x, (const bf16*)g,
                       (const bf16*)weight, (bf16*)y, rstd, rows, D, eps);
  return check_launch(fn);
}
