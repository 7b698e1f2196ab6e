// Chunked (WY / UT form) gated delta rule in fp32 arithmetic: q/k/v in fp32 or bf16, head sizes K == V of 64
// or 128, 64-token chunks. The path zgdn_chunk_fwd takes for everything but bf16 inputs at K == V == 128 (which
// gdn_chunk.hip runs on bf16 MFMA): the fp32 model dtype of lm.py:556-602, and 64-wide heads.
//
// Per chunk of L <= 64 tokens and value head h, with in-chunk cumulative log decay G (G_t = g_1 + .. + g_t; rows
// past L carry g = 0, beta = 0 and zero q, k, v, so G_L is G at row 63), start state S [V, K] (value-major) and
// scale s:
//   A   = strictly-lower( beta_i exp(G_i - G_j) k_i.k_j ),   T = (I + A)^-1             (unit lower triangular)
//   P   = s lower-incl( exp(G_i - G_j) q_i.k_j ),            R = P T diag(beta e^G)
//   W'  = diag(Fk) T diag(beta e^G) K,   Ub' = diag(Fk) T diag(beta) V,   Fk_t = exp(G_L - G_t)
//   Q'  = s diag(e^G) Q - R K,           Ob  = P T diag(beta) V
//   then, chunk after chunk:  U' = Ub' - W' S^T,  O = Ob + Q' S^T,  S <- e^{G_L} S + U'^T K
// (O = s diag(e^G) Q S^T + P (Ub - W S^T) and S_end = e^{G_L} S + sum_t e^{G_L - G_t} u_t k_t^T, the chunked
// statement of the token loop of lm.py:574-583.) Phase 1 (chunk32_prep_kernel) forms W', Q', K, Ub', Ob and G_L
// of every (chunk, value head) item at once; phase 2 (chunk32_state_kernel) walks each sequence's chunks in
// order. Every product runs on v_mfma_f32_16x16x4_f32 (fp32 operands and accumulation) and the q/k L2 norm,
// the gate and sigmoid(beta) are fp32, so the results follow the fp32 token loop to fp32 rounding.
//
// v_mfma_f32_16x16x4_f32, lane l = 16 g + m: A[m][g], B[g][m]; D[4 g + i][m] in element i. Four products
// i = 0..3 take the contraction indices 16 n + 4 g + i of a 16-wide block n, so that one 16-byte read of
// columns 16 n + 4 g .. + 3 of a row serves a lane for all four (for both operands when both are rows of
// row-major matrices), and a D tile is the B operand of the next product as it stands (a lane's element i
// is row 4 g + i of column m, the B element of product i).
//
// Matrices in LDS are fp32 row-major with the 16-byte chunk c of row r stored at chunk c ^ (r % 16): a
// 16-byte read of 16 consecutive rows at one column (the A operands) then meets every bank once, and so
// does a 4-byte read of 4 rows x 16 columns (the B operands read as columns).
#include <atomic>
#include <algorithm>

#include "gdn_common.h"

namespace zgdn {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// log(1 + e^x) with torch's threshold (identity above 20), full-precision exp and log1p.
__device__ __forceinline__ float softplus_exact(float x) { return x > 20.f ? x : log1pf(expf(x)); }

__device__ __forceinline__ f32x4 mma(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Byte offset of element (r, c) of a swizzled fp32 matrix with rows of RB bytes.
template <int RB>
__device__ __forceinline__ int swz(int r, int c) {
  return r * RB + ((((c >> 2) ^ (r & 15))) << 4) + ((c & 3) << 2);
}
__device__ __forceinline__ f32x4 ld4(const uint8_t* b, int off) { return *reinterpret_cast<const f32x4*>(b + off); }
__device__ __forceinline__ float ld1(const uint8_t* b, int off) { return *reinterpret_cast<const float*>(b + off); }
__device__ __forceinline__ void st4(uint8_t* b, int off, f32x4 v) { *reinterpret_cast<f32x4*>(b + off) = v; }
__device__ __forceinline__ void st1(uint8_t* b, int off, float v) { *reinterpret_cast<float*>(b + off) = v; }

// Workspace of one (chunk, value head) item, fp32, every block in the order phase 2 reads it (lane l = 16 g + m,
// token tile tt, key tile n, value tile vb, 64 lanes x 16 bytes = 1 KiB per block):
//   W'  [tt][n][l]: W'[16 tt + m][16 n + 4 g + i], i = 0..3       (A operands of W' S^T)
//   Q'  [tt][n][l]: Q'[16 tt + m][16 n + 4 g + i]                  (A operands of Q' S^T)
//   K^T [n][tt][l]: K[16 tt + 4 g + i][16 n + m]                    (A operands of the update U'^T K)
//   Ub' [vb][tt][l]: Ub'[16 tt + 4 g + i][16 vb + m]                 (D tiles: U' starts from them)
//   Ob  [vb][tt][l]: Ob[16 tt + 4 g + i][16 vb + m]                  (D tiles: O starts from them)
//   G_L (one float), padding to 256 bytes.
template <int D>
struct Ws32 {
  static constexpr int NK = D / 16;  // 16-wide key (and value) tiles
  static constexpr size_t BLK = (size_t)CHUNK_LEN * D * 4;
  static constexpr size_t W = 0, Q = BLK, K = 2 * BLK, U = 3 * BLK, O = 4 * BLK, G = 5 * BLK;
  static constexpr size_t ITEM = G + 256;
};

// ----------------------------------------------------------------------------------------------- phase 1
//
// One workgroup of 4 waves per item. LDS (byte offsets; D x 4-byte rows for the token rows, 256-byte rows for
// the 64 x 64 matrices): the chunk's q, k (L2-normalised in place when asked) and v rows, A (then R), T, P and
// the per-token factors.
template <int D>
struct Lds32 {
  static constexpr int RB = D * 4;
  static constexpr int K = 0, Q = 64 * RB, V = 2 * 64 * RB, A = 3 * 64 * RB, T = A + 16384, P = T + 16384;
  static constexpr int F = P + 16384;                                   // factors: 64 floats each
  static constexpr int FG = F, FB = F + 256, FEG = F + 512, FFK = F + 768, FBW = F + 1024;  // G, beta, e^G, Fk, beta e^G
  static constexpr int BYTES = F + 1280;
};

// Lower-triangle tile t (0..9) of a 4 x 4 block grid -> (row block, column block), row-major order.
__device__ __forceinline__ void tri_tile(int t, int& rb, int& cb) {
  rb = t < 1 ? 0 : (t < 3 ? 1 : (t < 6 ? 2 : 3));
  cb = t - rb * (rb + 1) / 2;
}

// 16 consecutive bytes of a q / k / v row as floats (4 fp32 or 8 bf16 elements).
__device__ __forceinline__ void load_vec(const float* p, float* out) {
  const f32x4 v = *reinterpret_cast<const f32x4*>(p);
  out[0] = v[0];
  out[1] = v[1];
  out[2] = v[2];
  out[3] = v[3];
}
__device__ __forceinline__ void load_vec(const bf16* p, float* out) {
  const uint4 w = *reinterpret_cast<const uint4*>(p);
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    out[2 * j] = __uint_as_float(u[j] << 16);
    out[2 * j + 1] = __uint_as_float(u[j] & 0xffff0000u);
  }
}

// acc += X[16 xr .., 16 xc ..] . Y[16 yr .., 16 yc ..] for 16 x 16 blocks of two 64 x 64 LDS matrices.
__device__ __forceinline__ f32x4 blk_mm(const uint8_t* lb, int xm, int xr, int xc, int ym, int yr, int yc, f32x4 acc) {
  const int l = threadIdx.x & 63, m = l & 15, g = l >> 4;
  const f32x4 a = ld4(lb, xm + swz<256>(16 * xr + m, 16 * xc + 4 * g));
#pragma unroll
  for (int i = 0; i < 4; ++i) acc = mma(a[i], ld1(lb, ym + swz<256>(16 * yr + 4 * g + i, 16 * yc + m)), acc);
  return acc;
}
// acc += X[16 xr .., 16 xc ..] . Y for a block Y held as a D tile.
__device__ __forceinline__ f32x4 blk_mm_d(const uint8_t* lb, int xm, int xr, int xc, f32x4 y, f32x4 acc) {
  const int l = threadIdx.x & 63, m = l & 15, g = l >> 4;
  const f32x4 a = ld4(lb, xm + swz<256>(16 * xr + m, 16 * xc + 4 * g));
#pragma unroll
  for (int i = 0; i < 4; ++i) acc = mma(a[i], y[i], acc);
  return acc;
}
// Stores a D tile as block (br, bc) of a 64 x 64 LDS matrix.
__device__ __forceinline__ void blk_put(uint8_t* lb, int mat, int br, int bc, f32x4 d) {
  const int l = threadIdx.x & 63, m = l & 15, g = l >> 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) st1(lb, mat + swz<256>(16 * br + 4 * g + i, 16 * bc + m), d[i]);
}

__device__ __forceinline__ void bar() { __syncthreads(); }

template <typename TIn, typename TG, int D, bool GATE>
__global__ __launch_bounds__(256) void chunk32_prep_kernel(
    const TIn* __restrict__ q, const TIn* __restrict__ k, const TIn* __restrict__ v, const TG* __restrict__ g,
    const TG* __restrict__ beta, const float* __restrict__ A_log, const float* __restrict__ dt_bias,
    const int32_t* __restrict__ cu, const int32_t* __restrict__ chunk_idx, int n_seqs, int T, int Hk, int Hv,
    float scale, int qk_l2norm, const RowStrides rs, uint8_t* __restrict__ ws) {
  using L = Lds32<D>;
  using WS = Ws32<D>;
  constexpr int RB = L::RB, NK = WS::NK, NKW = NK / 4;
  extern __shared__ f32x4 lds32[];
  uint8_t* lb = reinterpret_cast<uint8_t*>(lds32);
  const int tid = threadIdx.x, wave = wave_id(), l = tid & 63, m = l & 15, gq = l >> 4;
  const int item = blockIdx.x, c = item / Hv, h = item % Hv, hk = h / (Hv / Hk);
  const ChunkRange cr = chunk_range(c, cu, chunk_idx, T, n_seqs);
  uint8_t* out = ws + (size_t)item * WS::ITEM;

  // ---- rows of q, k (key head hk) and v (value head h) into LDS as fp32; zeros past the chunk end
  constexpr int VE = 16 / (int)sizeof(TIn), VPR = D / VE;
  for (int e = tid; e < 64 * VPR; e += 256) {
    const int r = e / VPR, c0 = (e % VPR) * VE;
    float xq[VE], xk[VE], xv[VE];
    if (r < cr.len) {
      const size_t t = (size_t)(cr.t0 + r);
      load_vec(q + t * rs.q + (size_t)hk * D + c0, xq);
      load_vec(k + t * rs.k + (size_t)hk * D + c0, xk);
      load_vec(v + t * rs.v + (size_t)h * D + c0, xv);
    } else {
#pragma unroll
      for (int j = 0; j < VE; ++j) xq[j] = xk[j] = xv[j] = 0.f;
    }
#pragma unroll
    for (int j = 0; j < VE; j += 4) {
      st4(lb, L::Q + swz<RB>(r, c0 + j), f32x4{xq[j], xq[j + 1], xq[j + 2], xq[j + 3]});
      st4(lb, L::K + swz<RB>(r, c0 + j), f32x4{xk[j], xk[j + 1], xk[j + 2], xk[j + 3]});
      st4(lb, L::V + swz<RB>(r, c0 + j), f32x4{xv[j], xv[j + 1], xv[j + 2], xv[j + 3]});
    }
  }
  // ---- per-token factors (wave 0, lane = token): g (the in-kernel gate when asked), beta, G = inclusive scan
  if (wave == 0) {
    float gt = 0.f, bt = 0.f;
    if (l < cr.len) {
      const size_t t = (size_t)(cr.t0 + l) * rs.gb + h;
      const float gr = io<TG>::load(g + t), br = io<TG>::load(beta + t);
      gt = GATE ? -expf(A_log[h]) * softplus_exact(gr + dt_bias[h]) : gr;
      bt = rs.beta_sigmoid ? 1.f / (1.f + expf(-br)) : br;
    }
    float G = gt;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const float o = __shfl_up(G, d, 64);
      if (l >= d) G += o;
    }
    const float GL = __shfl(G, 63, 64);
    const float eg = expf(G);
    st1(lb, L::FG + 4 * l, G);
    st1(lb, L::FB + 4 * l, bt);
    st1(lb, L::FEG + 4 * l, eg);
    st1(lb, L::FFK + 4 * l, expf(GL - G));
    st1(lb, L::FBW + 4 * l, bt * eg);
    if (l == 0) *reinterpret_cast<float*>(out + WS::G) = GL;
  }
  bar();
  // ---- q, k L2 norm in place: x * rsqrt(sum x^2 + 1e-6), 4 threads a row
  if (qk_l2norm) {
    const int r = tid >> 2, c0 = (tid & 3) * (D / 4);
    f32x4 xq[D / 16], xk[D / 16];
    float sq = 0.f, sk = 0.f;
#pragma unroll
    for (int j = 0; j < D / 16; ++j) {
      xq[j] = ld4(lb, L::Q + swz<RB>(r, c0 + 4 * j));
      xk[j] = ld4(lb, L::K + swz<RB>(r, c0 + 4 * j));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sq = fmaf(xq[j][e], xq[j][e], sq);
        sk = fmaf(xk[j][e], xk[j][e], sk);
      }
    }
    sq = group_sum<4>(sq);
    sk = group_sum<4>(sk);
    const float rq = 1.f / sqrtf(sq + 1e-6f), rk = 1.f / sqrtf(sk + 1e-6f);
#pragma unroll
    for (int j = 0; j < D / 16; ++j) {
      st4(lb, L::Q + swz<RB>(r, c0 + 4 * j), xq[j] * rq);
      st4(lb, L::K + swz<RB>(r, c0 + 4 * j), xk[j] * rk);
    }
    bar();
  }

  // ---- A = strictly-lower(beta_i e^{G_i - G_j} k_i.k_j), P = s lower-incl(e^{G_i - G_j} q_i.k_j): 20 tiles
  for (int u = wave; u < 20; u += 4) {
    const bool isP = u >= 10;
    int I, J;
    tri_tile(isP ? u - 10 : u, I, J);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int n = 0; n < NK; ++n) {
      const f32x4 a = ld4(lb, (isP ? L::Q : L::K) + swz<RB>(16 * I + m, 16 * n + 4 * gq));
      const f32x4 b = ld4(lb, L::K + swz<RB>(16 * J + m, 16 * n + 4 * gq));
#pragma unroll
      for (int i = 0; i < 4; ++i) acc = mma(a[i], b[i], acc);
    }
    const int cc = 16 * J + m;
    const float Gc = ld1(lb, L::FG + 4 * cc);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * I + 4 * gq + i;
      const float f = isP ? scale : ld1(lb, L::FB + 4 * r);
      const bool keep = isP ? r >= cc : r > cc;
      acc[i] = keep ? f * expf(ld1(lb, L::FG + 4 * r) - Gc) * acc[i] : 0.f;
    }
    blk_put(lb, isP ? L::P : L::A, I, J, acc);
  }
  bar();

  // ---- T = (I + A)^-1: diagonal blocks by substitution (wave d inverts block d; lane m holds column m)
  {
    const int d = wave;
    float x[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) x[r] = r == m ? 1.f : 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j)
#pragma unroll
      for (int r = j + 1; r < 16; ++r) x[r] = fmaf(-ld1(lb, L::A + swz<256>(16 * d + r, 16 * d + j)), x[j], x[r]);
    if (gq == 0) {
#pragma unroll
      for (int r = 0; r < 16; ++r) st1(lb, L::T + swz<256>(16 * d + r, 16 * d + m), x[r]);
    }
  }
  bar();
  // off-diagonal blocks, one level at a time: T_ij = -T_ii sum_{j <= m < i} A_im T_mj
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  if (wave < 3) {
    const int d = wave;
    const f32x4 y = blk_mm(lb, L::A, d + 1, d, L::T, d, d, z4);
    blk_put(lb, L::T, d + 1, d, -blk_mm_d(lb, L::T, d + 1, d + 1, y, z4));
  }
  bar();
  if (wave < 2) {
    const int d = wave;
    f32x4 y = blk_mm(lb, L::A, d + 2, d, L::T, d, d, z4);
    y = blk_mm(lb, L::A, d + 2, d + 1, L::T, d + 1, d, y);
    blk_put(lb, L::T, d + 2, d, -blk_mm_d(lb, L::T, d + 2, d + 2, y, z4));
  }
  bar();
  if (wave == 0) {
    f32x4 y = blk_mm(lb, L::A, 3, 0, L::T, 0, 0, z4);
    y = blk_mm(lb, L::A, 3, 1, L::T, 1, 0, y);
    y = blk_mm(lb, L::A, 3, 2, L::T, 2, 0, y);
    blk_put(lb, L::T, 3, 0, -blk_mm_d(lb, L::T, 3, 3, y, z4));
  }
  bar();

  // ---- R = P T diag(beta e^G) into A's place (tiles round-robin over the waves)
  for (int u = wave; u < 10; u += 4) {
    int I, J;
    tri_tile(u, I, J);
    f32x4 acc = z4;
    for (int M = J; M <= I; ++M) acc = blk_mm(lb, L::P, I, M, L::T, M, J, acc);
    acc *= ld1(lb, L::FBW + 4 * (16 * J + m));
    blk_put(lb, L::A, I, J, acc);
  }
  bar();

  // ---- W'^T and Q'^T (key tiles of this wave), with K^T: W'^T = K^T (diag(Fk) T diag(beta e^G))^T,
  //      Q'^T = s Q^T diag(e^G) - K^T R^T; each D tile is the phase-2 A operand block (tt = I, n)
#pragma unroll
  for (int j = 0; j < NKW; ++j) {
    const int n = wave * NKW + j;
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      const int tr = 16 * I + m;
      const float fk = ld1(lb, L::FFK + 4 * tr);
      f32x4 aw = z4;
      f32x4 aq = ld4(lb, L::Q + swz<RB>(tr, 16 * n + 4 * gq)) * (scale * ld1(lb, L::FEG + 4 * tr));
      for (int J = 0; J <= I; ++J) {
        const f32x4 t4 = ld4(lb, L::T + swz<256>(tr, 16 * J + 4 * gq));
        const f32x4 r4 = ld4(lb, L::A + swz<256>(tr, 16 * J + 4 * gq));
        const f32x4 bw = ld4(lb, L::FBW + 4 * (16 * J + 4 * gq));
        f32x4 kv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          kv[i] = ld1(lb, L::K + swz<RB>(16 * J + 4 * gq + i, 16 * n + m));
          aw = mma(kv[i], t4[i] * bw[i] * fk, aw);
          aq = mma(kv[i], -r4[i], aq);
        }
        if (I == 3) st4(out, (int)(WS::K + ((size_t)(n * 4 + J) * 64 + l) * 16), kv);
      }
      st4(out, (int)(WS::W + ((size_t)(I * NK + n) * 64 + l) * 16), aw);
      st4(out, (int)(WS::Q + ((size_t)(I * NK + n) * 64 + l) * 16), aq);
    }
  }
  // ---- Ub = T diag(beta) V and Ob = P Ub (value tiles of this wave); Ub' = diag(Fk) Ub
#pragma unroll
  for (int j = 0; j < NKW; ++j) {
    const int vb = wave * NKW + j;
    f32x4 ub[4];
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      f32x4 acc = z4;
      for (int J = 0; J <= I; ++J) {
        const f32x4 t4 = ld4(lb, L::T + swz<256>(16 * I + m, 16 * J + 4 * gq));
        const f32x4 b4 = ld4(lb, L::FB + 4 * (16 * J + 4 * gq));
#pragma unroll
        for (int i = 0; i < 4; ++i) acc = mma(t4[i] * b4[i], ld1(lb, L::V + swz<RB>(16 * J + 4 * gq + i, 16 * vb + m)), acc);
      }
      ub[I] = acc;
    }
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      f32x4 ob = z4;
#pragma unroll
      for (int J = 0; J <= I; ++J) ob = blk_mm_d(lb, L::P, I, J, ub[J], ob);
      const f32x4 fk = ld4(lb, L::FFK + 4 * (16 * I + 4 * gq));
      st4(out, (int)(WS::U + ((size_t)(vb * 4 + I) * 64 + l) * 16), ub[I] * fk);
      st4(out, (int)(WS::O + ((size_t)(vb * 4 + I) * 64 + l) * 16), ob);
    }
  }
}

// ----------------------------------------------------------------------------------------------- phase 2
//
// One workgroup of 4 waves per (sequence, value head, 16 value rows vb); wave w holds the state rows' key tiles
// n = w NK/4 .. as D tiles of S^T (lane: S[16 vb + m][16 n + 4 g + i]), which are the B operands of W' S^T and
// Q' S^T as they stand. Per chunk every wave forms its keys' part of W' S^T and Q' S^T for all 64 tokens and
// puts it in LDS; after one barrier each wave sums the four parts in wave order into U' = Ub' - W' S^T (all 64
// tokens: the B operands of its update), and wave w the outputs of token tile w. LDS buffers alternate by
// chunk, so one barrier a chunk suffices. The next chunk's operands are loaded while the current one computes.
template <int D>
struct Ops32 {
  static constexpr int NKW = D / 64;
  f32x4 W[4][NKW], Q[4][NKW], K[NKW][4], U[4], O;
  float GL;
};

template <int D>
__device__ __forceinline__ void load_ops(Ops32<D>& p, const uint8_t* base, int wave, int vb) {
  using WS = Ws32<D>;
  constexpr int NK = WS::NK, NKW = NK / 4;
  const int l = threadIdx.x & 63;
  auto at = [&](size_t off) { return *reinterpret_cast<const f32x4*>(base + off + (size_t)l * 16); };
#pragma unroll
  for (int j = 0; j < NKW; ++j) {
    const int n = wave * NKW + j;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      p.W[tt][j] = at(WS::W + (size_t)(tt * NK + n) * 1024);
      p.Q[tt][j] = at(WS::Q + (size_t)(tt * NK + n) * 1024);
      p.K[j][tt] = at(WS::K + (size_t)(n * 4 + tt) * 1024);
    }
  }
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) p.U[tt] = at(WS::U + (size_t)(vb * 4 + tt) * 1024);
  p.O = at(WS::O + (size_t)(vb * 4 + wave) * 1024);
  p.GL = *reinterpret_cast<const float*>(base + WS::G);
}

template <typename TOut, int D>
__global__ __launch_bounds__(256) void chunk32_state_kernel(const uint8_t* ws, const float* __restrict__ s_in,
                                                            float* __restrict__ s_out, TOut* __restrict__ o,
                                                            const int32_t* __restrict__ cu, int n_seqs,
                                                            int n_chunks, int T, int Hv) {
  using WS = Ws32<D>;
  constexpr int NK = WS::NK, NKW = NK / 4;
  // partial products of the 4 waves: [buffer][U', O][wave][token tile][lane]
  __shared__ f32x4 part[2][2][4][4][64];
  // the NK workgroups of one (sequence, head) share an id % 8, so they run on one XCD and share its L2 copy of
  // the chunk workspace (the grid is padded to whole groups of 8 NK)
  const int id = blockIdx.x;
  const int pair = (id / (8 * NK)) * 8 + id % 8, vb = (id % (8 * NK)) / 8;
  if (pair >= n_seqs * Hv) return;
  const int seq = pair / Hv, h = pair % Hv;
  const int wave = wave_id(), l = threadIdx.x & 63, m = l & 15, gq = l >> 4;
  int c0, bos, len;
  seq_chunks(cu, seq, T, c0, bos, len);
  // chunks past the workspace (a chunk table shorter than the sequences need) are not read
  const int nc = max(0, min((len + CHUNK_LEN - 1) / CHUNK_LEN, n_chunks - c0));

  const size_t srow = ((size_t)pair * D + 16 * vb + m) * D;  // this lane's state row
  f32x4 st[NKW];
#pragma unroll
  for (int j = 0; j < NKW; ++j) {
    const int col = 16 * (wave * NKW + j) + 4 * gq;
    st[j] = s_in != nullptr ? *reinterpret_cast<const f32x4*>(s_in + srow + col) : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  Ops32<D> cur;
  if (nc > 0) load_ops<D>(cur, ws + ((size_t)c0 * Hv + h) * WS::ITEM, wave, vb);
  for (int ci = 0; ci < nc; ++ci) {
    Ops32<D> nxt;
    load_ops<D>(nxt, ws + ((size_t)(c0 + min(ci + 1, nc - 1)) * Hv + h) * WS::ITEM, wave, vb);
    const int b = ci & 1;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      f32x4 pu = z4, po = z4;
#pragma unroll
      for (int j = 0; j < NKW; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pu = mma(cur.W[tt][j][i], st[j][i], pu);
          po = mma(cur.Q[tt][j][i], st[j][i], po);
        }
      part[b][0][wave][tt][l] = pu;
      part[b][1][wave][tt][l] = po;
    }
    __syncthreads();
    f32x4 u[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      u[tt] = cur.U[tt];
#pragma unroll
      for (int w = 0; w < 4; ++w) u[tt] -= part[b][0][w][tt][l];
    }
    f32x4 ov = cur.O;
#pragma unroll
    for (int w = 0; w < 4; ++w) ov += part[b][1][w][wave][l];
    // outputs of token tile `wave`: rows 16 wave + 4 g + i of column 16 vb + m
    const int tl = min(CHUNK_LEN, len - ci * CHUNK_LEN);
    const size_t t0 = (size_t)bos + (size_t)ci * CHUNK_LEN;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * wave + 4 * gq + i;
      if (r < tl) io<TOut>::store(o + ((t0 + r) * Hv + h) * D + 16 * vb + m, ov[i]);
    }
    // S^T <- e^{G_L} S^T + K^T U'
    const float gam = expf(cur.GL);
#pragma unroll
    for (int j = 0; j < NKW; ++j) {
      f32x4 acc = st[j] * gam;
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc = mma(cur.K[j][tt][i], u[tt][i], acc);
      st[j] = acc;
    }
    cur = nxt;
  }
  if (s_out != nullptr) {
#pragma unroll
    for (int j = 0; j < NKW; ++j)
      *reinterpret_cast<f32x4*>(s_out + srow + 16 * (wave * NKW + j) + 4 * gq) = st[j];
  }
}

// Phase 1's dynamic LDS is above the default 64 KiB at D = 128: raised once per device and kernel (the first
// call on that device); false when the device refuses.
constexpr int C32_MAX_DEVICES = 64;
template <typename K>
bool lds_ready(K kernel, int bytes, std::atomic<signed char>* state) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= C32_MAX_DEVICES) return false;
  const signed char s = state[dev].load(std::memory_order_acquire);
  if (s != 0) return s > 0;
  const bool ok = hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) ==
                  hipSuccess;
  if (!ok) (void)hipGetLastError();
  state[dev].store(ok ? 1 : -1, std::memory_order_release);
  return ok;
}

template <typename TIn, typename TG, int D, bool GATE>
int launch_prep32(const char* fn, int n_items, const void* q, const void* k, const void* v, const void* g,
                  const void* beta, const float* A_log, const float* dt_bias, const int32_t* cu,
                  const int32_t* chunk_idx, int n_seqs, int T, int Hk, int Hv, float scale, int qk_l2norm,
                  const RowStrides& rs, uint8_t* ws, hipStream_t s) {
  static std::atomic<signed char> state[C32_MAX_DEVICES];
  constexpr int bytes = Lds32<D>::BYTES;
  if (bytes > 65536 && !lds_ready(chunk32_prep_kernel<TIn, TG, D, GATE>, bytes, state))
    return fail(ZGDN_EHIP, "%s: the device refused %d bytes of LDS for the fp32 chunk kernel", fn, bytes);
  hipLaunchKernelGGL((chunk32_prep_kernel<TIn, TG, D, GATE>), dim3(n_items), dim3(256), bytes, s, (const TIn*)q, (const TIn*)k, (const TIn*)v,
                     (const TG*)g, (const TG*)beta, A_log, dt_bias, cu, chunk_idx, n_seqs, T, Hk, Hv, scale,
                     qk_l2norm, rs, ws);
  return ZGDN_OK;
}

template <typename TIn, int D>
int run32(const char* fn, int n_chunks, const void* q, const void* k, const void* v, const void* g, int gb_dtype,
          const void* beta, const float* A_log, const float* dt_bias, const int32_t* cu, const int32_t* chunk_idx,
          int N, int T, int Hk, int Hv, float scale, int qk_l2norm, const RowStrides& rs, const float* s_in,
          float* s_out, void* o, uint8_t* ws, hipStream_t s) {
  const int n_items = n_chunks * Hv;
  if (n_items > 0) {
    const bool gate = A_log != nullptr;
    int st;
    if (gb_dtype == ZGDN_F32)
      st = gate ? launch_prep32<TIn, float, D, true>(fn, n_items, q, k, v, g, beta, A_log, dt_bias, cu, chunk_idx, N,
                                                     T, Hk, Hv, scale, qk_l2norm, rs, ws, s)
                : launch_prep32<TIn, float, D, false>(fn, n_items, q, k, v, g, beta, A_log, dt_bias, cu, chunk_idx,
                                                      N, T, Hk, Hv, scale, qk_l2norm, rs, ws, s);
    else
      st = gate ? launch_prep32<TIn, bf16, D, true>(fn, n_items, q, k, v, g, beta, A_log, dt_bias, cu, chunk_idx, N,
                                                    T, Hk, Hv, scale, qk_l2norm, rs, ws, s)
                : launch_prep32<TIn, bf16, D, false>(fn, n_items, q, k, v, g, beta, A_log, dt_bias, cu, chunk_idx, N,
                                                     T, Hk, Hv, scale, qk_l2norm, rs, ws, s);
    if (st != ZGDN_OK) return st;
  }
  constexpr int NK = D / 16;
  const long pairs = (long)N * Hv;
  const dim3 grid((unsigned)(((pairs + 7) / 8) * 8 * NK));
  hipLaunchKernelGGL((chunk32_state_kernel<TIn, D>), grid, dim3(256), 0, s, ws, s_in, s_out, (TIn*)o, cu, N, n_chunks, T, Hv);
  return check_launch(fn);
}

}  // namespace

size_t chunk32_item_bytes(int D) { return D == 64 ? Ws32<64>::ITEM : Ws32<128>::ITEM; }

// The fp32-arithmetic chunked forward (arguments checked by the caller): q, k, v, o of element type qkv_dtype,
// K == V == D in {64, 128}; the workspace holds n_chunks * Hv items of chunk32_item_bytes(D).
int chunk32_fwd(const char* fn, const void* q, const void* k, const void* v, int qkv_dtype, const void* g,
                const void* beta, int gb_dtype, const float* A_log, const float* dt_bias, int qk_l2norm,
                const float* s_in, float* s_out, void* o, const int32_t* cu, const int32_t* chunk_idx, int N,
                int n_chunks, int T, int Hk, int Hv, int D, float scale, const RowStrides& rs, void* workspace,
                hipStream_t s) {
  uint8_t* ws = (uint8_t*)workspace;
#define ZGDN_RUN32(TIN, DD)                                                                                        \
  run32<TIN, DD>(fn, n_chunks, q, k, v, g, gb_dtype, beta, A_log, dt_bias, cu, chunk_idx, N, T, Hk, Hv, scale,    \
                 qk_l2norm, rs, s_in, s_out, o, ws, s)
  if (qkv_dtype == ZGDN_F32) return D == 64 ? ZGDN_RUN32(float, 64) : ZGDN_RUN32(float, 128);
  return D == 64 ? ZGDN_RUN32(bf16, 64) : ZGDN_RUN32(bf16, 128);
#undef ZGDN_RUN32
}

}  // namespace zgdn
