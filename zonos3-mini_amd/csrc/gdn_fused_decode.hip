// Fused single-token GDN block for a batch of streams: causal conv1d (width 4, rolling cache) + SiLU, q/k
// L2-norm, in-kernel gate, gated delta-rule state update and the gated RMSNorm of the output, in one launch.
//
// The reference statement is model/src/zonos3/reference/lm.py:563-587 applied to one new row per stream:
//   conv   = silu(conv1d([history | x]))       computed in fp32, rounded to the input dtype after the conv and
//                                              after the SiLU (F.conv1d / F.silu on x.dtype tensors)
//   q, k   = l2norm(conv_q), l2norm(conv_k)    fp32, x * rsqrt(sum x^2 + 1e-6)
//   decay  = exp(-exp(A_log) softplus(a + dt_bias)), beta = sigmoid(b)
//   S      = decay S; d = beta (v - S k); S += d k^T; o = S (q scale)     (fp32 state [Hv, V, K])
//   out    = (rms_norm(o.to(dtype)) * w).to(dtype) * silu(z), product in fp32, cast to dtype
// Value head h reads key head h / (Hv / Hk) (servers/mlx/src/zonos3_mlx/models/gdn_kernel.py:16-18).
//
// Work layout: one workgroup per (stream, key head): it owns the G = Hv / Hk value heads that share the key
// head, so the q/k conv-cache rows it rewrites are read by no other workgroup. Its 8 waves first issue the
// loads of their state rows (G * 128 rows of 512 B), then form the conv / norms / gates of the group in LDS,
// then update the rows exactly like the recurrent kernel (16 lanes per row, DPP row reductions) and finish
// with the per-head gated RMSNorm.
#include "gdn_common.h"

namespace zgdn {
namespace {

constexpr int FD_WAVES = 8;
constexpr int FD_K = 128;   // key / value head size
constexpr int FD_W = 4;     // conv width
constexpr int FD_LPR = FD_K / 8;             // lanes per state row
constexpr int FD_RPP = 64 / FD_LPR;          // rows per wave pass (4)
constexpr int FD_ROWS_PASS = FD_RPP * FD_WAVES;  // rows per workgroup pass (32)

template <typename T>
__device__ __forceinline__ float round_to(float x) {
  if constexpr (sizeof(T) == 2) return bf16_to_f32(f32_to_bf16(x));
  else return x;
}

template <typename T, int G>
__global__ __launch_bounds__(64 * FD_WAVES) void fused_decode_kernel(
    const T* __restrict__ x, const T* __restrict__ z, const T* __restrict__ a, const T* __restrict__ b,
    const T* __restrict__ conv_w, T* __restrict__ conv_cache, const float* __restrict__ A_log,
    const float* __restrict__ dt_bias, const T* __restrict__ norm_w, float* __restrict__ state, T* __restrict__ out,
    int Hk, int Hv, float eps, float scale) {
  constexpr int PASSES = G * FD_K / FD_ROWS_PASS;  // 4 per value head
  constexpr int NCH = 2 * FD_K + G * FD_K;         // conv channels of the group
  __shared__ float s_conv[NCH];                    // q | k | v_0 .. v_{G-1} after conv + SiLU (+ L2 for q, k)
  __shared__ float s_o[G][FD_K];
  __shared__ float s_red[FD_WAVES][1];
  __shared__ float s_gate[G][2];

  const int bs = blockIdx.x / Hk, hk = blockIdx.x % Hk;
  const int C = 2 * Hk * FD_K + Hv * FD_K;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int sub = lane % FD_LPR, rsub = lane / FD_LPR;
  const int c0 = sub * 4, c1 = FD_K / 2 + sub * 4;

  // 0. issue the state loads of this lane's rows (row r = pass * 32 + wave * 4 + rsub; head r / 128)
  float* sgroup = state + ((size_t)bs * Hv + (size_t)hk * G) * FD_K * FD_K;
  float s[PASSES][8];
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int r = p * FD_ROWS_PASS + wave * FD_RPP + rsub;
    const float* src = sgroup + (size_t)r * FD_K;
    const float4 u = io<float>::load4(src + c0), w = io<float>::load4(src + c1);
    s[p][0] = u.x; s[p][1] = u.y; s[p][2] = u.z; s[p][3] = u.w;
    s[p][4] = w.x; s[p][5] = w.y; s[p][6] = w.z; s[p][7] = w.w;
  }

  // 1. conv + SiLU of the group's channels; the rolling history becomes (h1, h2, x)
  for (int i = tid; i < NCH; i += 64 * FD_WAVES) {
    int ch;
    if (i < FD_K) ch = hk * FD_K + i;                                     // q
    else if (i < 2 * FD_K) ch = Hk * FD_K + hk * FD_K + (i - FD_K);       // k
    else ch = 2 * Hk * FD_K + hk * G * FD_K + (i - 2 * FD_K);             // v of heads hk*G ..
    const size_t xc = (size_t)bs * C + ch;
    T* hist = conv_cache + xc * (FD_W - 1);
    const float xv = io<T>::load(x + xc);
    const float h0 = io<T>::load(hist), h1 = io<T>::load(hist + 1), h2 = io<T>::load(hist + 2);
    const T* w = conv_w + (size_t)ch * FD_W;
    float acc = io<T>::load(w) * h0;
    acc = fmaf(io<T>::load(w + 1), h1, acc);
    acc = fmaf(io<T>::load(w + 2), h2, acc);
    acc = fmaf(io<T>::load(w + 3), xv, acc);
    s_conv[i] = round_to<T>(silu(round_to<T>(acc)));
    io<T>::store(hist, h1);
    io<T>::store(hist + 1, h2);
    io<T>::store(hist + 2, xv);
  }
  if (tid < G) {
    const int h = hk * G + tid;
    const size_t gi = (size_t)bs * Hv + h;
    s_gate[tid][0] = __expf(-__expf(A_log[h]) * softplus(io<T>::load(a + gi) + dt_bias[h]));
    s_gate[tid][1] = sigmoid(io<T>::load(b + gi));
  }
  __syncthreads();

  // 2. L2 norms of q (wave 0) and k (wave 1): 2 values per lane
  if (wave < 2) {
    float* v = s_conv + wave * FD_K;
    const float x0 = v[lane], x1 = v[lane + 64];
    const float ss = wave_sum(x0 * x0 + x1 * x1);
    const float r = rsqrtf(ss + 1e-6f);
    v[lane] = x0 * r;
    v[lane + 64] = x1 * r;
  }
  __syncthreads();

  // 3. delta-rule update of the rows
  float kk[8], qq[8];
  {
    const float4 ka = *reinterpret_cast<const float4*>(s_conv + FD_K + c0);
    const float4 kb = *reinterpret_cast<const float4*>(s_conv + FD_K + c1);
    const float4 qa = *reinterpret_cast<const float4*>(s_conv + c0);
    const float4 qb = *reinterpret_cast<const float4*>(s_conv + c1);
    kk[0] = ka.x; kk[1] = ka.y; kk[2] = ka.z; kk[3] = ka.w; kk[4] = kb.x; kk[5] = kb.y; kk[6] = kb.z; kk[7] = kb.w;
    qq[0] = qa.x; qq[1] = qa.y; qq[2] = qa.z; qq[3] = qa.w; qq[4] = qb.x; qq[5] = qb.y; qq[6] = qb.z; qq[7] = qb.w;
  }
  float kq = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) kq = fmaf(kk[i], qq[i], kq);
  kq = group_sum<FD_LPR>(kq);
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int r = p * FD_ROWS_PASS + wave * FD_RPP + rsub;
    const int g = r / FD_K, j = r % FD_K;
    const float alpha = s_gate[g][0], bt = s_gate[g][1];
    const float vj = s_conv[2 * FD_K + r];
    float pk = 0.f, pq = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      pk = fmaf(s[p][i], kk[i], pk);
      pq = fmaf(s[p][i], qq[i], pq);
    }
    pk = group_sum<FD_LPR>(pk);
    pq = group_sum<FD_LPR>(pq);
    const float delta = bt * (vj - alpha * pk);
#pragma unroll
    for (int i = 0; i < 8; ++i) s[p][i] = fmaf(delta, kk[i], alpha * s[p][i]);
    float* dst = sgroup + (size_t)r * FD_K;
    io<float>::store4(dst + c0, make_float4(s[p][0], s[p][1], s[p][2], s[p][3]));
    io<float>::store4(dst + c1, make_float4(s[p][4], s[p][5], s[p][6], s[p][7]));
    if (sub == 0) s_o[g][j] = scale * fmaf(delta, kq, alpha * pq);
  }
  __syncthreads();

  // 4. gated RMSNorm per value head: waves 2g, 2g+1 own head g (128 values, one per thread)
  if (wave < 2 * G) {
    const int g = wave >> 1, j = tid - g * FD_K;
    const float ov = round_to<T>(s_o[g][j]);
    const float sq = wave_sum(ov * ov);
    if (lane == 0) s_red[wave][0] = sq;
  }
  __syncthreads();
  if (wave < 2 * G) {
    const int g = wave >> 1, j = tid - g * FD_K;
    const int h = hk * G + g;
    const float ov = round_to<T>(s_o[g][j]);
    const float ms = (s_red[2 * g][0] + s_red[2 * g + 1][0]) / (float)FD_K;
    const float nrm = round_to<T>(ov * rsqrtf(ms + eps) * io<T>::load(norm_w + j));
    const size_t zi = ((size_t)bs * Hv + h) * FD_K + j;
    io<T>::store(out + zi, nrm * silu(io<T>::load(z + zi)));
  }
}

template <typename T>
void launch_fused(int G, int B, int Hk, int Hv, const void* x, const void* z, const void* a, const void* b,
                  const void* conv_w, void* conv_cache, const float* A_log, const float* dt_bias, const void* norm_w,
                  float* state, void* out, float eps, float scale, hipStream_t stream) {
  dim3 grid(B * Hk), block(64 * FD_WAVES);
#define ZGDN_FUSED_CASE(GG)                                                                                     \
  case GG:                                                                                                      \
    hipLaunchKernelGGL((fused_decode_kernel<T, GG>), grid, block, 0, stream, (const T*)x, (const T*)z,         \
                       (const T*)a, (const T*)b, (const T*)conv_w, (T*)conv_cache, A_log, dt_bias,             \
                       (const T*)norm_w, state, (T*)out, Hk, Hv, eps, scale);                                  \
    break;
  switch (G) {
    ZGDN_FUSED_CASE(1)
    ZGDN_FUSED_CASE(2)
    ZGDN_FUSED_CASE(4)
  }
#undef ZGDN_FUSED_CASE
}

}  // namespace
}  // namespace zgdn

extern "C" int zgdn_fused_decode_step(const void* x_qkv, const void* z, const void* a, const void* b, int dtype,
                                      const void* conv_weight, void* conv_cache, const float* A_log,
                                      const float* dt_bias, const void* norm_weight, float* state, void* out,
                                      int B, int Hk, int Hv, int K, int V, int W, float eps, float scale,
                                      void* stream) {
  using namespace zgdn;
  const char* fn = "zgdn_fused_decode_step";
  if (!x_qkv || !z || !a || !b || !conv_weight || !conv_cache || !A_log || !dt_bias || !norm_weight || !state ||
      !out)
    return fail(ZGDN_EINVAL, "%s: null pointer", fn);
  if (K != FD_K || V != FD_K) return fail(ZGDN_EUNSUPPORTED, "%s: K=%d V=%d (supported: 128)", fn, K, V);
  if (W != FD_W) return fail(ZGDN_EUNSUPPORTED, "%s: conv width %d (supported: 4)", fn, W);
  if (B < 1 || Hk < 1 || Hv < 1 || Hv % Hk) return fail(ZGDN_EINVAL, "%s: bad sizes B=%d Hk=%d Hv=%d", fn, B, Hk, Hv);
  const int G = Hv / Hk;
  if (G != 1 && G != 2 && G != 4) return fail(ZGDN_EUNSUPPORTED, "%s: Hv/Hk=%d (supported: 1, 2, 4)", fn, G);
  if (dtype != ZGDN_F32 && dtype != ZGDN_BF16) return fail(ZGDN_EINVAL, "%s: dtype code %d", fn, dtype);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ZGDN_F32)
    launch_fused<float>(G, B, Hk, Hv, x_qkv, z, a, b, conv_weight, conv_cache, A_log, dt_bias, norm_weight, state,
                        out, eps, scale, s);
  else
    launch_fused<bf16>(G, B, Hk, Hv, x_qkv, z, a, b, conv_weight, conv_cache, A_log, dt_bias, norm_weight, state,
                       out, eps, scale, s);
  return check_launch(fn);
}
