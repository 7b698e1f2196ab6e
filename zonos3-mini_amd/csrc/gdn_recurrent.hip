// Recurrent gated delta rule (token-by-token), including the single-token decode step.
//
// Layout of the work: the value-major state [N, Hv, V, K] splits into independent rows S[n, h, j, :] (one
// value index j each). A row of K fp32 is held by LPR = K/8 lanes of a wave, 8 floats per lane, as two
// 16-byte pieces at columns c..c+3 and K/2+c..K/2+c+3 (c = 4 * lane-in-row), so each 128-bit load or store
// instruction of a wave covers 64/LPR rows' contiguous halves. A wave walks PASSES such row groups; the
// state stays in registers across tokens and is read and written exactly once per call with 128-bit
// accesses (ordinary ones: on gfx950 the non-temporal forms measured slower for this stream). Row dot
// products reduce over the LPR lanes with DPP.
//
// Per token and row (lm.py:574-583 rewritten with one read of S):
//   pk = S.k, pq = S.q (S before decay), alpha = exp(g)
//   delta = beta (v_j - alpha pk)
//   S <- alpha S + delta k
//   o_j = scale (alpha pq + delta (k.q))            (== S_new . q scale)
#include <algorithm>

#include "gdn_common.h"

namespace zgdn {
namespace {

// Default tiling: PASSES row groups per wave, NWAVES waves per workgroup.
#ifndef ZGDN_REC_PASSES
#define ZGDN_REC_PASSES 1
#endif
#ifndef ZGDN_REC_NWAVES
#define ZGDN_REC_NWAVES 8
#endif

template <typename TIn, typename TOut, typename TG, int K, int PASSES = ZGDN_REC_PASSES,
          int NWAVES = ZGDN_REC_NWAVES>
__global__ __launch_bounds__(64 * NWAVES) void recurrent_kernel(
    const TIn* __restrict__ q, const TIn* __restrict__ k, const TIn* __restrict__ v, const TG* __restrict__ g,
    const TG* __restrict__ beta, const float* __restrict__ A_log, const float* __restrict__ dt_bias, int qk_l2norm,
    const float* s_in, float* s_out, TOut* __restrict__ o, const int32_t* __restrict__ cu, int T, int Hk, int Hv,
    int V, float scale) {
  constexpr int LPR = K / 8;         // lanes per state row
  constexpr int RPP = 64 / LPR;      // rows per pass of a wave
  constexpr int ROWS_WAVE = RPP * PASSES;
  constexpr int ROWS_WG = ROWS_WAVE * NWAVES;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sub = lane % LPR;
  const int rsub = lane / LPR;
  const int c0 = sub * 4;
  const int c1 = K / 2 + sub * 4;

  const int n = blockIdx.z;
  const int h = blockIdx.y;
  const int hk = h / (Hv / Hk);
  int bos, eos;
  if (cu != nullptr) {
    seq_bounds(cu, n, T, bos, eos);
  } else {
    bos = n * T;
    eos = bos + T;
  }
  const int row0 = blockIdx.x * ROWS_WG + wave * ROWS_WAVE + rsub;

  float s[PASSES][8];
  const size_t head_base = ((size_t)n * Hv + h) * (size_t)V;
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int row = row0 + p * RPP;
    if (s_in != nullptr && row < V) {
      const float* src = s_in + (head_base + row) * K;
      float4 a = io<float>::load4(src + c0);
      float4 b = io<float>::load4(src + c1);
      s[p][0] = a.x; s[p][1] = a.y; s[p][2] = a.z; s[p][3] = a.w;
      s[p][4] = b.x; s[p][5] = b.y; s[p][6] = b.z; s[p][7] = b.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) s[p][i] = 0.f;
    }
  }

  for (int t = bos; t < eos; ++t) {
    const size_t qk_off = ((size_t)t * Hk + hk) * K;
    float4 ka = io<TIn>::load4(k + qk_off + c0), kb = io<TIn>::load4(k + qk_off + c1);
    float4 qa = io<TIn>::load4(q + qk_off + c0), qb = io<TIn>::load4(q + qk_off + c1);
    float kk[8] = {ka.x, ka.y, ka.z, ka.w, kb.x, kb.y, kb.z, kb.w};
    float qq[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    if (qk_l2norm) {  // x * rsqrt(sum x^2 + 1e-6) in fp32 (lm.py:570-571)
      float nk = 0.f, nq = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        nk = fmaf(kk[i], kk[i], nk);
        nq = fmaf(qq[i], qq[i], nq);
      }
      const float rk = rsqrtf(group_sum<LPR>(nk) + 1e-6f), rq = rsqrtf(group_sum<LPR>(nq) + 1e-6f);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        kk[i] *= rk;
        qq[i] *= rq;
      }
    }
    const size_t gh = (size_t)t * Hv + h;
    const float graw = io<TG>::load(g + gh);
    // in-kernel gate (lm.py:572): log decay = -exp(A_log) softplus(a + dt_bias); otherwise g is the log decay
    const float alpha = __expf(A_log != nullptr ? -__expf(A_log[h]) * softplus(graw + dt_bias[h]) : graw);
    const float bt = io<TG>::load(beta + gh);
    float kq = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) kq = fmaf(kk[i], qq[i], kq);
    kq = group_sum<LPR>(kq);
    const size_t v_base = gh * (size_t)V;
    float vj[PASSES];
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int row = row0 + p * RPP;
      const float x = io<TIn>::load(v + v_base + min(row, V - 1));  // clamped: no divergent load
      vj[p] = row < V ? x : 0.f;
    }
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int row = row0 + p * RPP;
      float pk = 0.f, pq = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        pk = fmaf(s[p][i], kk[i], pk);
        pq = fmaf(s[p][i], qq[i], pq);
      }
      pk = group_sum<LPR>(pk);
      pq = group_sum<LPR>(pq);
      const float delta = bt * (vj[p] - alpha * pk);
#pragma unroll
      for (int i = 0; i < 8; ++i) s[p][i] = fmaf(delta, kk[i], alpha * s[p][i]);
      if (sub == 0 && row < V) io<TOut>::store(o + v_base + row, scale * fmaf(delta, kq, alpha * pq));
    }
  }

  if (s_out != nullptr) {
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int row = row0 + p * RPP;
      if (row < V) {
        float* dst = s_out + (head_base + row) * K;
        io<float>::store4(dst + c0, make_float4(s[p][0], s[p][1], s[p][2], s[p][3]));
        io<float>::store4(dst + c1, make_float4(s[p][4], s[p][5], s[p][6], s[p][7]));
      }
    }
  }
}

// ------------------------------------------------------------------------------ single-token step (T == 1)
//
// One token per stream is one pass over the state, so the step is a stream of state rows with no reuse: the
// kernel is persistent and software-pipelined. Work is split into tiles of GPT row groups (RPP rows each, one
// row per LPR lanes, the register layout above) of one (stream, head), so a tile's q/k row, g and beta are
// loaded once for GPT groups. Each wave walks tiles gridDim.x * STEP_NWAVES apart and issues the next tile's
// loads (state rows, q/k row, v, g, beta) before it updates and stores the current tile, so a tile's reads
// are always in flight while the wave computes and writes. Loads keep the raw input words and convert when
// used, so issuing them never waits for data. The prefetch after a wave's last tile is clamped to the last
// tile (an unused read) so that every iteration waits on the same, exact count of outstanding loads. The LEAN
// form is the plain decode step (state read and written, g the log decay, q/k as given, V a multiple of the
// tile's rows): its loads are all unconditional, so the compiler's wait counts stay exact; the other form
// takes every option of the entry point.

template <typename T>
struct raw4;  // four consecutive inputs as loaded, and as floats
template <>
struct raw4<float> {
  using type = float4;
  __device__ __forceinline__ static type load(const float* p) { return *reinterpret_cast<const float4*>(p); }
  __device__ __forceinline__ static void unpack(type w, float* f) { f[0] = w.x; f[1] = w.y; f[2] = w.z; f[3] = w.w; }
};
template <>
struct raw4<bf16> {
  using type = uint2;
  __device__ __forceinline__ static type load(const bf16* p) { return *reinterpret_cast<const uint2*>(p); }
  __device__ __forceinline__ static void unpack(type w, float* f) {
    f[0] = __uint_as_float(w.x << 16); f[1] = __uint_as_float(w.x & 0xffff0000u);
    f[2] = __uint_as_float(w.y << 16); f[3] = __uint_as_float(w.y & 0xffff0000u);
  }
};
__device__ __forceinline__ float as_f32(float x) { return x; }
__device__ __forceinline__ float as_f32(bf16 x) { return bf16_to_f32(x.bits); }

template <typename TIn, typename TG, int GPT>
struct StepTile {
  float4 s[GPT][2];                                    // the lane's 8 state entries of its row in each group
  typename raw4<TIn>::type ka, kb, qa, qb;             // the lane's 8 entries of k and q
  TIn vj[GPT];
  TG g, beta;
  float a_log, dt_bias;
};

constexpr int STEP_NWAVES = 4;

template <typename TIn, typename TOut, typename TG, int K, bool LEAN, int GPT>
__global__ __launch_bounds__(64 * STEP_NWAVES) void step_kernel(
    const TIn* __restrict__ q, const TIn* __restrict__ k, const TIn* __restrict__ v, const TG* __restrict__ g,
    const TG* __restrict__ beta, const float* __restrict__ A_log, const float* __restrict__ dt_bias, int qk_l2norm,
    const float* s_in, float* s_out, TOut* __restrict__ o, int n_tiles, int Hk, int Hv, int V, float scale) {
  constexpr int LPR = K / 8, RPP = 64 / LPR, ROWS = RPP * GPT;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % LPR, rsub = lane / LPR;
  const int c0 = sub * 4, c1 = K / 2 + sub * 4;
  const int tph = (V + ROWS - 1) / ROWS;  // tiles per (stream, head)
  using Tile = StepTile<TIn, TG, GPT>;

  auto load = [&](int ti, Tile& x) {
    const int nh = ti / tph;  // stream * Hv + head: also the token row of g, beta, v
    const int n = nh / Hv, h = nh - n * Hv, hk = h / (Hv / Hk);
    const int row0 = (ti - nh * tph) * ROWS + rsub;
#pragma unroll
    for (int j = 0; j < GPT; ++j) {
      int row = row0 + j * RPP;
      if constexpr (!LEAN) row = min(row, V - 1);  // clamped: no divergent load
      if (LEAN || s_in != nullptr) {
        const float* src = s_in + ((size_t)nh * V + row) * K;
        x.s[j][0] = *reinterpret_cast<const float4*>(src + c0);
        x.s[j][1] = *reinterpret_cast<const float4*>(src + c1);
      } else {
        x.s[j][0] = x.s[j][1] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    const size_t qk = ((size_t)n * Hk + hk) * K;
    x.ka = raw4<TIn>::load(k + qk + c0);
    x.kb = raw4<TIn>::load(k + qk + c1);
    x.qa = raw4<TIn>::load(q + qk + c0);
    x.qb = raw4<TIn>::load(q + qk + c1);
#pragma unroll
    for (int j = 0; j < GPT; ++j) {
      int row = row0 + j * RPP;
      if constexpr (!LEAN) row = min(row, V - 1);
      x.vj[j] = v[(size_t)nh * V + row];
    }
    x.g = g[nh];
    x.beta = beta[nh];
    if (!LEAN && A_log != nullptr) {
      x.a_log = A_log[h];
      x.dt_bias = dt_bias[h];
    }
  };

  auto process = [&](int ti, const Tile& x) {
    const int nh = ti / tph, row0 = (ti - nh * tph) * ROWS + rsub;
    float kk[8], qq[8];
    raw4<TIn>::unpack(x.ka, kk);
    raw4<TIn>::unpack(x.kb, kk + 4);
    raw4<TIn>::unpack(x.qa, qq);
    raw4<TIn>::unpack(x.qb, qq + 4);
    if (!LEAN && qk_l2norm) {  // x * rsqrt(sum x^2 + 1e-6) in fp32 (lm.py:570-571)
      float nk = 0.f, nq = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        nk = fmaf(kk[i], kk[i], nk);
        nq = fmaf(qq[i], qq[i], nq);
      }
      const float rk = rsqrtf(group_sum<LPR>(nk) + 1e-6f), rq = rsqrtf(group_sum<LPR>(nq) + 1e-6f);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        kk[i] *= rk;
        qq[i] *= rq;
      }
    }
    const float graw = as_f32(x.g);
    const float alpha = __expf(!LEAN && A_log != nullptr ? -__expf(x.a_log) * softplus(graw + x.dt_bias) : graw);
    const float bt = as_f32(x.beta);
    float kq = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) kq = fmaf(kk[i], qq[i], kq);
    kq = group_sum<LPR>(kq);
#pragma unroll
    for (int j = 0; j < GPT; ++j) {
      const int row = row0 + j * RPP;
      float st[8] = {x.s[j][0].x, x.s[j][0].y, x.s[j][0].z, x.s[j][0].w,
                     x.s[j][1].x, x.s[j][1].y, x.s[j][1].z, x.s[j][1].w};
      float pk = 0.f, pq = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        pk = fmaf(st[i], kk[i], pk);
        pq = fmaf(st[i], qq[i], pq);
      }
      pk = group_sum<LPR>(pk);
      pq = group_sum<LPR>(pq);
      const float delta = bt * (as_f32(x.vj[j]) - alpha * pk);
#pragma unroll
      for (int i = 0; i < 8; ++i) st[i] = fmaf(delta, kk[i], alpha * st[i]);
      if (LEAN || row < V) {
        if (sub == 0) io<TOut>::store(o + (size_t)nh * V + row, scale * fmaf(delta, kq, alpha * pq));
        if (LEAN || s_out != nullptr) {
          float* dst = s_out + ((size_t)nh * V + row) * K;
          *reinterpret_cast<float4*>(dst + c0) = make_float4(st[0], st[1], st[2], st[3]);
          *reinterpret_cast<float4*>(dst + c1) = make_float4(st[4], st[5], st[6], st[7]);
        }
      }
    }
  };

  const int stride = gridDim.x * STEP_NWAVES;
  int ti = blockIdx.x * STEP_NWAVES + wave;
  if (ti >= n_tiles) return;
  const int last = n_tiles - 1;
  Tile b0, b1;
  load(ti, b0);
  if (stride >= n_tiles) {  // one item per wave: nothing to prefetch
    process(ti, b0);
    return;
  }
  for (;;) {  // two buffers in turn; every wave leaves after its last tile
    const int t1 = ti + stride;
    load(min(t1, last), b1);
    process(ti, b0);
    if (t1 >= n_tiles) break;
    const int t2 = t1 + stride;
    load(min(t2, last), b0);
    process(t1, b1);
    if (t2 >= n_tiles) break;
    ti = t2;
  }
}

struct RecArgs {
  const void *q, *k, *v, *g, *beta;
  const float *A_log, *dt_bias;
  int qk_l2norm;
  const float* s_in;
  float* s_out;
  void* o;
  const int32_t* cu;
  int N, T, Hk, Hv, V;
  float scale;
};

// The single-token step: lean 4-group tiles where there are enough of them for STEP_TILE_WGS_PER_CU
// workgroups on every CU (about 128 VGPRs: 4 waves per SIMD; 3 workgroups per CU measured fastest), single
// groups otherwise (small batches, where more waves in flight matter more than q/k reuse) and for the general
// form, with as many workgroups as fit on a CU at once.
constexpr int STEP_TILE_WGS_PER_CU = 3;

template <typename TIn, typename TOut, typename TG, int K>
bool launch_step(const RecArgs& a, hipStream_t stream) {
  constexpr int RPP = 64 / (K / 8);
  const long long groups = (long long)a.N * a.Hv * ((a.V + RPP - 1) / RPP);
  if (groups > INT32_MAX) return false;
  int dev = 0, n_cu = 256;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    n_cu = 256;
  n_cu = std::max(1, n_cu);
  const bool lean = a.s_in != nullptr && a.s_out != nullptr && a.A_log == nullptr && !a.qk_l2norm &&
                    a.V % RPP == 0;
  const long long tiles4 = (long long)a.N * a.Hv * (a.V / (4 * RPP));
  const bool tiled = lean && a.V % (4 * RPP) == 0 && tiles4 >= (long long)STEP_TILE_WGS_PER_CU * n_cu * STEP_NWAVES;
  const long long n_tiles = tiled ? tiles4 : groups;
  auto kernel = tiled  ? step_kernel<TIn, TOut, TG, K, true, 4>
                : lean ? step_kernel<TIn, TOut, TG, K, true, 1>
                       : step_kernel<TIn, TOut, TG, K, false, 1>;
  int per_cu = STEP_TILE_WGS_PER_CU;
  if (!tiled && (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 64 * STEP_NWAVES, 0) != hipSuccess ||
                 per_cu < 1))
    per_cu = 4;
  const long long all = (n_tiles + STEP_NWAVES - 1) / STEP_NWAVES;  // one item per wave
  long long wgs = std::min<long long>(all, (long long)per_cu * n_cu);
  // single groups: up to two per resident wave would leave some waves one behind the others for a whole
  // group's latency; one group per wave (the hardware queues the rest) finishes sooner there (B=16, H=16)
  if (!tiled && all <= 2LL * per_cu * n_cu) wgs = all;
  hipLaunchKernelGGL(kernel, dim3((unsigned)wgs), dim3(64 * STEP_NWAVES), 0, stream, (const TIn*)a.q,
                     (const TIn*)a.k, (const TIn*)a.v, (const TG*)a.g, (const TG*)a.beta, a.A_log, a.dt_bias,
                     a.qk_l2norm, a.s_in, a.s_out, (TOut*)a.o, (int)n_tiles, a.Hk, a.Hv, a.V, a.scale);
  return true;
}

template <typename TIn, typename TOut, typename TG, int K>
void launch(const RecArgs& a, hipStream_t stream) {
  if (a.T == 1 && a.cu == nullptr && launch_step<TIn, TOut, TG, K>(a, stream)) return;
  constexpr int PASSES = ZGDN_REC_PASSES, NWAVES = ZGDN_REC_NWAVES;
  constexpr int ROWS_WG = (64 / (K / 8)) * PASSES * NWAVES;
  dim3 grid((a.V + ROWS_WG - 1) / ROWS_WG, a.Hv, a.N);
  hipLaunchKernelGGL((recurrent_kernel<TIn, TOut, TG, K>), grid, dim3(64 * NWAVES), 0, stream,
                     (const TIn*)a.q, (const TIn*)a.k, (const TIn*)a.v, (const TG*)a.g, (const TG*)a.beta, a.A_log,
                     a.dt_bias, a.qk_l2norm, a.s_in, a.s_out, (TOut*)a.o, a.cu, a.T, a.Hk, a.Hv, a.V, a.scale);
}

template <typename TIn, typename TOut, typename TG>
void launch_k(int K, const RecArgs& a, hipStream_t stream) {
  if (K == 128)
    launch<TIn, TOut, TG, 128>(a, stream);
  else
    launch<TIn, TOut, TG, 64>(a, stream);
}

template <typename TIn, typename TOut>
void launch_g(int gb_dtype, int K, const RecArgs& a, hipStream_t stream) {
  if (gb_dtype == ZGDN_F32)
    launch_k<TIn, TOut, float>(K, a, stream);
  else
    launch_k<TIn, TOut, bf16>(K, a, stream);
}

}  // namespace
}  // namespace zgdn

extern "C" int zgdn_recurrent_fwd(const void* q, const void* k, const void* v, int qkv_dtype, const void* g,
                                  const void* beta, int gb_dtype, const float* A_log, const float* dt_bias,
                                  int qk_l2norm, const float* initial_state, float* final_state, void* o,
                                  int o_dtype, const int32_t* cu_seqlens, int n_seqs, int B, int T, int Hk, int Hv,
                                  int K, int V, float scale, void* stream) {
  using namespace zgdn;
  const char* fn = "zgdn_recurrent_fwd";
  if (!q || !k || !v || !g || !beta || !o) return fail(ZGDN_EINVAL, "%s: null tensor pointer", fn);
  if (B < 1 || T < 0 || Hk < 1 || Hv < 1 || V < 1)
    return fail(ZGDN_EINVAL, "%s: bad sizes B=%d T=%d Hk=%d Hv=%d V=%d", fn, B, T, Hk, Hv, V);
  if (Hv % Hk) return fail(ZGDN_EINVAL, "%s: Hv=%d is not a multiple of Hk=%d", fn, Hv, Hk);
  if (K != 64 && K != 128) return fail(ZGDN_EUNSUPPORTED, "%s: K=%d (supported: 64, 128)", fn, K);
  if ((A_log == nullptr) != (dt_bias == nullptr)) return fail(ZGDN_EINVAL, "%s: A_log and dt_bias go together", fn);
  for (int dt : {qkv_dtype, gb_dtype, o_dtype})
    if (dt != ZGDN_F32 && dt != ZGDN_BF16) return fail(ZGDN_EINVAL, "%s: unknown dtype code %d", fn, dt);
  int N = B;
  if (cu_seqlens != nullptr) {
    if (B != 1) return fail(ZGDN_EINVAL, "%s: cu_seqlens needs B == 1 (got B=%d)", fn, B);
    if (n_seqs < 1) return fail(ZGDN_EINVAL, "%s: n_seqs=%d with cu_seqlens", fn, n_seqs);
    N = n_seqs;
  }
  RecArgs a{q, k, v, g, beta, A_log, dt_bias, qk_l2norm, initial_state, final_state, o, cu_seqlens, N, T, Hk, Hv,
            V, scale};
  hipStream_t s = (hipStream_t)stream;
  if (qkv_dtype == ZGDN_F32 && o_dtype == ZGDN_F32)
    launch_g<float, float>(gb_dtype, K, a, s);
  else if (qkv_dtype == ZGDN_F32)
    launch_g<float, bf16>(gb_dtype, K, a, s);
  else if (o_dtype == ZGDN_F32)
    launch_g<bf16, float>(gb_dtype, K, a, s);
  else
    launch_g<bf16, bf16>(gb_dtype, K, a, s);
  return check_launch(fn);
}
