// Fused single-token GDN block for a batch of streams: causal conv1d (width 4, rolling cache) + SiLU, q/k
// L2-norm, in-kernel gate, gated delta-rule state update and the gated RMSNorm of the output, in one launch.
//
// The reference statement is model/src/zonos3/reference/lm.py:563-587 applied to one new row per stream:
//   conv   = silu(conv1d([history | x]))       computed in fp32, rounded to the input dtype after the conv and
//                                              after the SiLU (F.conv1d / F.silu on x.dtype tensors)
//   q, k   = l2norm(conv_q), l2norm(conv_k)    fp32, x * rsqrt(sum x^2 + 1e-6); with qk_round rounded to the
//                                              input dtype, as the serving layer's l2norm operator returns
//                                              them (servers/sgl/src/zonos3_sgl/models/gdn.py:416-417)
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
#include <type_traits>

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

// Where a launch reads and writes. The plain block step: stream b's rows at b, conv cache [B, C, W-1].
// The serving step: stream b's q|k|v, z, a, b are slices of one in_proj row, its caches are those of table
// slot slots[b] (conv history [cap, C, W], the FLA layout), and a window that fills up commits the new
// conv history and state to the committed caches.
template <typename T>
struct FusedArgs {
  const T* x;          // q|k|v channels of stream b at x + b * x_ld
  const T* z;          // z of stream b at z + b * z_ld, [Hv, V]
  const T* a;          // a, b of stream b at a/b + b * ab_ld, [Hv]
  const T* b;
  long x_ld, z_ld, ab_ld;
  const T* conv_w;     // [C, W]
  T* conv_cache;       // [rows, C, CW]: the last CW raw inputs, oldest first
  const float* A_log;
  const float* dt_bias;
  const T* norm_w;
  float* state;        // [rows, Hv, V, K]
  T* out;              // [B, Hv, V]
  const int64_t* slots;     // serving: rows of stream b; rows outside [0, n_rows) are skipped (else row b), and
                            // so is every stream whose slot an earlier stream of the batch already holds
  long n_rows;
  int32_t* win_len;         // serving: real rows in each slot's window, advanced by the step (see the kernel)
  T* conv_commit;           // serving: committed caches, written when the window fills
  float* state_commit;
  T* window;                // serving: [rows, window_rows, hidden] raw rows; receives stream b's row
  const T* x_hidden;        // [B, hidden]
  int hidden, window_rows;
  int Hk, Hv;
  float eps, scale;
  int qk_round;
};

// Channel of the group's i-th conv channel: q, k of key head hk, then the v of value heads hk*G ..
__device__ __forceinline__ int conv_channel(int i, int hk, int Hk, int G) {
  if (i < FD_K) return hk * FD_K + i;
  if (i < 2 * FD_K) return Hk * FD_K + hk * FD_K + (i - FD_K);
  return 2 * Hk * FD_K + hk * G * FD_K + (i - 2 * FD_K);
}

template <typename T, int G, int CW>
__global__ __launch_bounds__(64 * FD_WAVES) void fused_decode_kernel(const FusedArgs<T> p) {
  constexpr bool SERVING = CW == FD_W;  // slot-indexed caches, window and commits (the serving step)
  constexpr int PASSES = G * FD_K / FD_ROWS_PASS;  // 4 per value head
  constexpr int NCH = 2 * FD_K + G * FD_K;         // conv channels of the group
  __shared__ float s_conv[NCH];                    // q | k | v_0 .. v_{G-1} after conv + SiLU (+ L2 for q, k)
  __shared__ float s_o[G][FD_K];
  __shared__ float s_red[FD_WAVES][1];
  __shared__ float s_gate[G][2];
  __shared__ int s_wlen;

  const int Hk = p.Hk, Hv = p.Hv;
  const int bs = blockIdx.x / Hk, hk = blockIdx.x % Hk;
  long srow = bs;
  if constexpr (SERVING) {
    srow = p.slots[bs];
    if (srow < 0 || srow >= p.n_rows) return;  // a slot outside the caches: nothing is read or written
    // A slot named again later in the batch (padded graph replays repeat one spare slot) is served by its
    // first stream only: the later ones read and write nothing, so every slot sees exactly Hk arrivals below
    // and its window-length word keeps only the length.
    int dup = 0;
    for (int i = threadIdx.x; i < bs; i += blockDim.x) dup |= p.slots[i] == srow;
    if (__syncthreads_or(dup)) return;
  }
  const size_t row = (size_t)srow;
  const int C = 2 * Hk * FD_K + Hv * FD_K;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int sub = lane % FD_LPR, rsub = lane / FD_LPR;
  const int c0 = sub * 4, c1 = FD_K / 2 + sub * 4;
  // 0. issue the state loads of this lane's rows (row r = pass * 32 + wave * 4 + rsub; head r / 128)
  const size_t group_off = (row * Hv + (size_t)hk * G) * FD_K * FD_K;
  float* sgroup = p.state + group_off;
  float s[PASSES][8];
#pragma unroll
  for (int q = 0; q < PASSES; ++q) {
    const int r = q * FD_ROWS_PASS + wave * FD_RPP + rsub;
    const float* src = sgroup + (size_t)r * FD_K;
    const float4 u = io<float>::load4(src + c0), w = io<float>::load4(src + c1);
    s[q][0] = u.x; s[q][1] = u.y; s[q][2] = u.z; s[q][3] = u.w;
    s[q][4] = w.x; s[q][5] = w.y; s[q][6] = w.z; s[q][7] = w.w;
  }
  // The slot's window length, advanced in the same launch: workgroup hk of the slot adds 1 << 16 (an arrival
  // count above the length, which stays below 2^16) and takes the length from the low bits of the old value;
  // the last of the slot's Hk arrivals stores the new length (win_len + 1) % window_rows with the count
  // cleared, so the word holds only the length once the launch ends. The atomic is issued here and its value
  // is waited for only at the barrier that ends step 1.
  int old_len = 0;
  if (SERVING && tid == 0)
    old_len = __hip_atomic_fetch_add(p.win_len + row, 1 << 16, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // 1. conv + SiLU of the group's channels; the history rolls by one (the oldest input drops out)
  for (int i = tid; i < NCH; i += 64 * FD_WAVES) {
    const int ch = conv_channel(i, hk, Hk, G);
    const size_t hc = (row * C + ch) * CW;
    T* hist = p.conv_cache + hc + (CW - (FD_W - 1));  // the taps' history: the last W-1 columns
    const float xv = io<T>::load(p.x + bs * p.x_ld + ch);
    const float h0 = io<T>::load(hist), h1 = io<T>::load(hist + 1), h2 = io<T>::load(hist + 2);
    const T* w = p.conv_w + (size_t)ch * FD_W;
    float acc = io<T>::load(w) * h0;
    acc = fmaf(io<T>::load(w + 1), h1, acc);
    acc = fmaf(io<T>::load(w + 2), h2, acc);
    acc = fmaf(io<T>::load(w + 3), xv, acc);
    s_conv[i] = round_to<T>(silu(round_to<T>(acc)));
    T* dst = p.conv_cache + hc;
    if constexpr (CW == FD_W) io<T>::store(dst++, h0);  // a full-width history keeps h0 as its oldest input
    io<T>::store(dst, h1);
    io<T>::store(dst + 1, h2);
    io<T>::store(dst + 2, xv);
  }
  if (tid < G) {
    const int h = hk * G + tid;
    s_gate[tid][0] = __expf(-__expf(p.A_log[h]) * softplus(io<T>::load(p.a + bs * p.ab_ld + h) + p.dt_bias[h]));
    s_gate[tid][1] = sigmoid(io<T>::load(p.b + bs * p.ab_ld + h));
  }
  if (SERVING && tid == 0) {
    s_wlen = old_len & 0xffff;
    if ((old_len >> 16) == Hk - 1)
      __hip_atomic_store(p.win_len + row, (s_wlen + 1) % p.window_rows, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  bool commit = false;
  if constexpr (SERVING) {
    const int wlen = s_wlen;
    commit = wlen + 1 == p.window_rows;
    if (hk == 0 && wlen < p.window_rows) {  // the raw row joins the slot's window
      T* wrow = p.window + (row * p.window_rows + wlen) * p.hidden;
      const T* xrow = p.x_hidden + (size_t)bs * p.hidden;
      for (int i = tid; i < p.hidden; i += 64 * FD_WAVES) wrow[i] = xrow[i];
    }
    if (commit) {  // a full window commits the new conv history (this thread's own stores of step 1)
      for (int i = tid; i < NCH; i += 64 * FD_WAVES) {
        const size_t hc = (row * C + conv_channel(i, hk, Hk, G)) * CW;
        for (int c = 0; c < CW; ++c) p.conv_commit[hc + c] = p.conv_cache[hc + c];
      }
    }
  }

  // 2. L2 norms of q (wave 0) and k (wave 1): 2 values per lane
  if (wave < 2) {
    float* v = s_conv + wave * FD_K;
    const float x0 = v[lane], x1 = v[lane + 64];
    const float ss = wave_sum(x0 * x0 + x1 * x1);
    const float r = rsqrtf(ss + 1e-6f);
    v[lane] = p.qk_round ? round_to<T>(x0 * r) : x0 * r;
    v[lane + 64] = p.qk_round ? round_to<T>(x1 * r) : x1 * r;
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
  for (int q = 0; q < PASSES; ++q) {
    const int r = q * FD_ROWS_PASS + wave * FD_RPP + rsub;
    const int g = r / FD_K, j = r % FD_K;
    const float alpha = s_gate[g][0], bt = s_gate[g][1];
    const float vj = s_conv[2 * FD_K + r];
    float pk = 0.f, pq = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      pk = fmaf(s[q][i], kk[i], pk);
      pq = fmaf(s[q][i], qq[i], pq);
    }
    pk = group_sum<FD_LPR>(pk);
    pq = group_sum<FD_LPR>(pq);
    const float delta = bt * (vj - alpha * pk);
#pragma unroll
    for (int i = 0; i < 8; ++i) s[q][i] = fmaf(delta, kk[i], alpha * s[q][i]);
    const float4 n0 = make_float4(s[q][0], s[q][1], s[q][2], s[q][3]);
    const float4 n1 = make_float4(s[q][4], s[q][5], s[q][6], s[q][7]);
    float* dst = sgroup + (size_t)r * FD_K;
    io<float>::store4(dst + c0, n0);
    io<float>::store4(dst + c1, n1);
    if (SERVING && commit) {
      float* cdst = p.state_commit + group_off + (size_t)r * FD_K;
      io<float>::store4(cdst + c0, n0);
      io<float>::store4(cdst + c1, n1);
    }
    if (sub == 0) s_o[g][j] = p.scale * fmaf(delta, kq, alpha * pq);
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
    const float nrm = round_to<T>(ov * rsqrtf(ms + p.eps) * io<T>::load(p.norm_w + j));
    const float zv = io<T>::load(p.z + bs * p.z_ld + (size_t)h * FD_K + j);
    io<T>::store(p.out + ((size_t)bs * Hv + h) * FD_K + j, nrm * silu(zv));
  }
}

template <typename T, int CW>
void launch_fused(int G, int B, const FusedArgs<T>& p, hipStream_t stream) {
  dim3 grid(B * p.Hk), block(64 * FD_WAVES);
  switch (G) {
    case 1: hipLaunchKernelGGL((fused_decode_kernel<T, 1, CW>), grid, block, 0, stream, p); break;
    case 2: hipLaunchKernelGGL((fused_decode_kernel<T, 2, CW>), grid, block, 0, stream, p); break;
    case 4: hipLaunchKernelGGL((fused_decode_kernel<T, 4, CW>), grid, block, 0, stream, p); break;
  }
}

int check_fused_sizes(const char* fn, int B, int Hk, int Hv, int K, int V, int W, int dtype) {
  if (K != FD_K || V != FD_K) return fail(ZGDN_EUNSUPPORTED, "%s: K=%d V=%d (supported: 128)", fn, K, V);
  if (W != FD_W) return fail(ZGDN_EUNSUPPORTED, "%s: conv width %d (supported: 4)", fn, W);
  if (B < 1 || Hk < 1 || Hv < 1 || Hv % Hk) return fail(ZGDN_EINVAL, "%s: bad sizes B=%d Hk=%d Hv=%d", fn, B, Hk, Hv);
  const int G = Hv / Hk;
  if (G != 1 && G != 2 && G != 4) return fail(ZGDN_EUNSUPPORTED, "%s: Hv/Hk=%d (supported: 1, 2, 4)", fn, G);
  if (dtype != ZGDN_F32 && dtype != ZGDN_BF16) return fail(ZGDN_EINVAL, "%s: dtype code %d", fn, dtype);
  return ZGDN_OK;
}

template <typename T>
FusedArgs<T> plain_args(const void* x_qkv, const void* z, const void* a, const void* b, const void* conv_weight,
                        void* conv_cache, const float* A_log, const float* dt_bias, const void* norm_weight,
                        float* state, void* out, int Hk, int Hv, float eps, float scale, int qk_round) {
  FusedArgs<T> p{};
  p.x = (const T*)x_qkv;
  p.z = (const T*)z;
  p.a = (const T*)a;
  p.b = (const T*)b;
  p.x_ld = 2L * Hk * FD_K + (long)Hv * FD_K;
  p.z_ld = (long)Hv * FD_K;
  p.ab_ld = Hv;
  p.conv_w = (const T*)conv_weight;
  p.conv_cache = (T*)conv_cache;
  p.A_log = A_log;
  p.dt_bias = dt_bias;
  p.norm_w = (const T*)norm_weight;
  p.state = state;
  p.out = (T*)out;
  p.Hk = Hk;
  p.Hv = Hv;
  p.eps = eps;
  p.scale = scale;
  p.qk_round = qk_round;
  return p;
}

}  // namespace
}  // namespace zgdn

extern "C" int zgdn_fused_decode_step(const void* x_qkv, const void* z, const void* a, const void* b, int dtype,
                                      const void* conv_weight, void* conv_cache, const float* A_log,
                                      const float* dt_bias, const void* norm_weight, float* state, void* out,
                                      int B, int Hk, int Hv, int K, int V, int W, float eps, float scale,
                                      int qk_round, void* stream) {
  using namespace zgdn;
  const char* fn = "zgdn_fused_decode_step";
  if (!x_qkv || !z || !a || !b || !conv_weight || !conv_cache || !A_log || !dt_bias || !norm_weight || !state ||
      !out)
    return fail(ZGDN_EINVAL, "%s: null pointer", fn);
  if (int rc = check_fused_sizes(fn, B, Hk, Hv, K, V, W, dtype)) return rc;
  const int G = Hv / Hk;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == ZGDN_F32)
    launch_fused<float, FD_W - 1>(G, B, plain_args<float>(x_qkv, z, a, b, conv_weight, conv_cache, A_log, dt_bias,
                                                          norm_weight, state, out, Hk, Hv, eps, scale, qk_round), s);
  else
    launch_fused<bf16, FD_W - 1>(G, B, plain_args<bf16>(x_qkv, z, a, b, conv_weight, conv_cache, A_log, dt_bias,
                                                        norm_weight, state, out, Hk, Hv, eps, scale, qk_round), s);
  return check_launch(fn);
}

extern "C" int zgdn_serving_decode_step(const void* mixed, long mixed_ld, const void* x_hidden, int hidden,
                                        int dtype, const int64_t* slots, int n_slots, int B, int Hk, int Hv, int K,
                                        int V, int W,
                                        const void* conv_weight, void* conv_live, void* conv_commit,
                                        float* state_live, float* state_commit, void* window, int32_t* win_len,
                                        int window_rows, const float* A_log, const float* dt_bias,
                                        const void* norm_weight, void* out, float eps, float scale, int qk_round,
                                        void* stream) {
  using namespace zgdn;
  const char* fn = "zgdn_serving_decode_step";
  if (!mixed || !x_hidden || !slots || !conv_weight || !conv_live || !conv_commit || !state_live ||
      !state_commit || !window || !win_len || !A_log || !dt_bias || !norm_weight || !out)
    return fail(ZGDN_EINVAL, "%s: null pointer", fn);
  if (int rc = check_fused_sizes(fn, B, Hk, Hv, K, V, W, dtype)) return rc;
  const long C = 2L * Hk * K + (long)Hv * V;
  if (mixed_ld < C + (long)Hv * V + 2L * Hv)
    return fail(ZGDN_EINVAL, "%s: in_proj row of %ld elements holds no q|k|v (%ld), z (%d), a, b (%d each)", fn,
                mixed_ld, C, Hv * V, Hv);
  if (hidden < 1 || window_rows < 1 || n_slots < 1)
    return fail(ZGDN_EINVAL, "%s: hidden=%d window_rows=%d n_slots=%d", fn, hidden, window_rows, n_slots);
  const int G = Hv / Hk;
  hipStream_t s = (hipStream_t)stream;
  auto fill = [&](auto* tag) {
    using T = std::remove_pointer_t<decltype(tag)>;
    FusedArgs<T> p{};
    p.x = (const T*)mixed;
    p.z = p.x + C;
    p.a = p.z + (long)Hv * V;
    p.b = p.a + Hv;
    p.x_ld = p.z_ld = p.ab_ld = mixed_ld;
    p.conv_w = (const T*)conv_weight;
    p.conv_cache = (T*)conv_live;
    p.A_log = A_log;
    p.dt_bias = dt_bias;
    p.norm_w = (const T*)norm_weight;
    p.state = state_live;
    p.out = (T*)out;
    p.slots = slots;
    p.n_rows = n_slots;
    p.win_len = win_len;
    p.conv_commit = (T*)conv_commit;
    p.state_commit = state_commit;
    p.window = (T*)window;
    p.x_hidden = (const T*)x_hidden;
    p.hidden = hidden;
    p.window_rows = window_rows;
    p.Hk = Hk;
    p.Hv = Hv;
    p.eps = eps;
    p.scale = scale;
    p.qk_round = qk_round;
    launch_fused<T, FD_W>(G, B, p, s);
  };
  if (window_rows >= (1 << 16))
    return fail(ZGDN_EUNSUPPORTED, "%s: window_rows=%d (the step keeps the length below 2^16)", fn, window_rows);
  if (dtype == ZGDN_F32)
    fill((float*)nullptr);
  else
    fill((bf16*)nullptr);
  return check_launch(fn);
}
