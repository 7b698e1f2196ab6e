// Chunked (WY / UT form) gated delta rule prefill on bf16 MFMA, 64-token chunks, dk = dv = 128.
//
// Per chunk of L <= 64 tokens and value head h, with in-chunk cumulative log decay G (G_i = g_1+..+g_i), start
// state S0 [V, K] (value-major) and scale s (derivation: the chunked statement of the oracle):
//   A  = strictly-lower( beta_i exp(G_i - G_j) k_i.k_j )           T = (I + A)^-1   (unit lower triangular)
//   W  = T diag(beta exp(G)) K                                      [L x K]
//   Ub = diag(beta) V + (T - I) diag(beta) V                        [L x V]   (diagonal exact in fp32)
//   P  = s * lower-incl( exp(G_i - G_j) q_i.k_j )                   [L x L]
//   Qp = s diag(exp(G)) Q - P W,    Ol = P Ub
//   U  = Ub - W S0^T                (the corrected values)
//   O  = Ol + Qp S0^T
//   S  = exp(G_L) S0 + (diag(exp(G_L - G)) U)^T K
// Phase 1 (chunk_prep_kernel, one workgroup per chunk x head, all independent) forms Qp, W, Ub, Ol and K^T
// into a workspace. Phase 2 (chunk_state_kernel, one workgroup per sequence x head x 16 value rows) walks the
// chunks in order keeping its 16 x 128 slice of the fp32 state in registers: U = Ub - W S^T and O = Ol + Qp S^T
// are one MFMA pass over [Qp; W], the state update is a second. Numerics: MFMA operands are bf16 with fp32
// accumulation; the decayed U enters the state update as a hi + lo bf16 pair (two MFMAs), and the diagonal
// of T diag(beta) is applied in fp32, which keeps the fp32 state within ~1e-4 of the exact recurrence.
//
// MFMA used: v_mfma_f32_16x16x32_bf16 (A: row lane%16, k 8*(lane/16)+0..7; B: column lane%16, same k;
// D: row 4*(lane/16)+i, column lane%16) and v_mfma_f32_16x16x4_f32 (A[lane%16][lane/16], B[lane/16][lane%16])
// for the fp32 block inverse.
#include "gdn_common.h"

namespace zgdn {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int CH = 64;    // chunk length
constexpr int DK = 128;   // key dim
constexpr int DV = 128;   // value dim
constexpr int VB = 16;    // value rows per phase-2 workgroup
constexpr int LDQ = DK + 8;  // padded LDS row (bf16) of a 128-wide matrix
constexpr int LDC = CH + 8;  // padded LDS row (bf16) of a 64-wide matrix
constexpr int LDF = CH + 4;  // padded LDS row (fp32) of a 64-wide matrix

// Workspace of one chunk x head (bytes).
constexpr size_t WS_QP = 0;                                 // Qp [64][128] bf16
constexpr size_t WS_W = WS_QP + CH * DK * 2;                // W  [64][128] bf16
constexpr size_t WS_KT = WS_W + CH * DK * 2;                // K^T [128][64] bf16
constexpr size_t WS_UT = WS_KT + DK * CH * 2;               // Ub^T [128][64] fp32
constexpr size_t WS_OT = WS_UT + DV * CH * 4;               // Ol^T [128][64] bf16
constexpr size_t WS_G = WS_OT + DV * CH * 2;                // G [64] fp32
constexpr size_t WS_CHUNK = WS_G + CH * 4;                  // 98,560 bytes

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// 8 consecutive bf16 of row (r0 + lane%16), columns k0 + 8*(lane/16) .. +7, of a row-major bf16 matrix.
__device__ __forceinline__ bf16x8 frag(const uint16_t* base, int ld, int r0, int k0) {
  const int l = lane_id();
  return *reinterpret_cast<const bf16x8*>(base + (r0 + (l & 15)) * ld + k0 + 8 * (l >> 4));
}

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// Tile (r0.., c0..) of A . B where A is row-major [.][lda] and B is given by its transpose Bt [.][ldb],
// contraction over k in [0, kend) (kend a multiple of 32).
__device__ __forceinline__ f32x4 tile_mm(const uint16_t* A, int lda, int r0, const uint16_t* Bt, int ldb, int c0,
                                         int kend, f32x4 acc) {
  for (int k0 = 0; k0 < kend; k0 += 32) acc = mfma(frag(A, lda, r0, k0), frag(Bt, ldb, c0, k0), acc);
  return acc;
}

// 16x16x16 fp32 block product acc += A[16][16] . B[16][16] (row-major fp32 in LDS).
__device__ __forceinline__ f32x4 mm16_f32(const float* A, int lda, const float* B, int ldb, f32x4 acc) {
  const int l = lane_id();
#pragma unroll
  for (int s = 0; s < 4; ++s)
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(A[(l & 15) * lda + 4 * s + (l >> 4)],
                                                B[(4 * s + (l >> 4)) * ldb + (l & 15)], acc, 0, 0, 0);
  return acc;
}

template <typename T>
__device__ __forceinline__ void load8(const T* p, float* out);
template <>
__device__ __forceinline__ void load8<bf16>(const bf16* p, float* out) {
  uint4 w = *reinterpret_cast<const uint4*>(p);
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(u[i] << 16);
    out[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
  }
}
template <>
__device__ __forceinline__ void load8<float>(const float* p, float* out) {
  float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
  out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w; out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
}

// Token range of chunk `c`: packed sequences (cu != nullptr, chunk index table (seq, j)) or B x T batches.
struct ChunkRange {
  int t0, len;
};
__device__ __forceinline__ ChunkRange chunk_range(int c, const int32_t* cu, const int32_t* chunk_idx, int T,
                                                  int n_seqs) {
  ChunkRange r;
  if (cu != nullptr) {
    const int s = chunk_idx[2 * c], j = chunk_idx[2 * c + 1];
    if (s < 0 || s >= n_seqs || j < 0) {  // a malformed table row reads nothing
      r.t0 = 0;
      r.len = 0;
      return r;
    }
    const int bos = cu[s], eos = cu[s + 1];
    r.t0 = bos + j * CH;
    r.len = min(CH, eos - r.t0);
  } else {
    const int nt = (T + CH - 1) / CH;
    const int b = c / nt, j = c % nt;
    r.t0 = b * T + j * CH;
    r.len = min(CH, T - j * CH);
  }
  return r;
}

// ----------------------------------------------------------------------------------------------- phase 1

constexpr int P1_WAVES = 8;

struct Prep {
  uint16_t KsT[DK][LDC];      // K^T   (B operand of W = TB K)
  uint16_t VsT[DV][LDC];      // V^T   (B operand of Ub = LB V)
  union {
    struct {
      uint16_t Qs[CH][LDQ];   // Q, K rows (A/B operands of K K^T, Q K^T)
      uint16_t Ks[CH][LDQ];
    } a;
    struct {
      uint16_t WsT[DK][LDC];  // W^T, Ub^T (B operands of P W, P Ub)
      uint16_t UsT[DV][LDC];
    } d;
  } u;
  float As[CH][LDF];          // strictly lower A (fp32)
  float Ts[CH][LDF];          // T = (I + A)^-1 (fp32)
  float Ys[P1_WAVES][16][20];  // per-wave 16x16 fp32 scratch of the block inverse
  uint16_t Ps[CH][LDC];       // P (bf16), A operand of P W and P Ub
  uint16_t TBs[CH][LDC];      // T diag(beta exp G)
  uint16_t LBs[CH][LDC];      // (T - I) diag(beta)
  float Gs[CH];
  float Bs[CH];
};

template <typename TIn, typename TG, bool GATE>
__global__ __launch_bounds__(64 * P1_WAVES) void chunk_prep_kernel(
    const TIn* __restrict__ q, const TIn* __restrict__ k, const TIn* __restrict__ v, const TG* __restrict__ g,
    const TG* __restrict__ beta, const float* __restrict__ A_log, const float* __restrict__ dt_bias,
    const int32_t* __restrict__ cu, const int32_t* __restrict__ chunk_idx, int n_seqs, int T, int Hk, int Hv,
    float scale, uint8_t* __restrict__ ws) {
  __shared__ Prep sm;
  const int c = blockIdx.x, h = blockIdx.y;
  const int hk = h / (Hv / Hk);
  const int tid = threadIdx.x, l = lane_id(), wave = tid >> 6;
  const ChunkRange cr = chunk_range(c, cu, chunk_idx, T, n_seqs);
  uint8_t* wsc = ws + ((size_t)c * Hv + h) * WS_CHUNK;

  // 1. q, k, v rows -> LDS (zero rows past the chunk end); K^T and V^T transposed copies.
  for (int e = tid; e < CH * (DK / 8); e += 64 * P1_WAVES) {
    const int r = e / (DK / 8), c8 = (e % (DK / 8)) * 8;
    float qf[8], kf[8], vf[8];
    if (r < cr.len) {
      const size_t t = (size_t)(cr.t0 + r);
      load8<TIn>(q + (t * Hk + hk) * DK + c8, qf);
      load8<TIn>(k + (t * Hk + hk) * DK + c8, kf);
      load8<TIn>(v + (t * Hv + h) * DV + c8, vf);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) qf[i] = kf[i] = vf[i] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint16_t qb = f32_to_bf16(qf[i]), kb = f32_to_bf16(kf[i]), vb = f32_to_bf16(vf[i]);
      sm.u.a.Qs[r][c8 + i] = qb;
      sm.u.a.Ks[r][c8 + i] = kb;
      sm.KsT[c8 + i][r] = kb;
      sm.VsT[c8 + i][r] = vb;
    }
  }
  if (wave == 0) {
    float gi = 0.f, bi = 0.f;
    if (l < cr.len) {
      const size_t gh = (size_t)(cr.t0 + l) * Hv + h;
      gi = io<TG>::load(g + gh);
      if constexpr (GATE) gi = -__expf(A_log[h]) * softplus(gi + dt_bias[h]);
      bi = io<TG>::load(beta + gh);
    }
    // inclusive prefix sum over the 64 lanes
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const float o = __shfl_up(gi, d);
      if (l >= d) gi += o;
    }
    sm.Gs[l] = gi;
    sm.Bs[l] = bi;
    reinterpret_cast<float*>(wsc + WS_G)[l] = gi;
  }
  __syncthreads();

  // 2. K K^T and Q K^T on the lower block triangle (10 tiles each): A and P.
  f32x4 acc[3];
  int jobs[3];
  int njob = 0;
  for (int job = wave; job < 20; job += P1_WAVES) {
    const int which = job / 10, t = job % 10;  // t -> (rb, cb) with rb >= cb
    int rb = 0;
    while ((rb + 1) * (rb + 2) / 2 <= t) ++rb;
    const int cb = t - rb * (rb + 1) / 2;
    const uint16_t* Am = which ? &sm.u.a.Qs[0][0] : &sm.u.a.Ks[0][0];
    acc[njob] = tile_mm(Am, LDQ, rb * 16, &sm.u.a.Ks[0][0], LDQ, cb * 16, DK, zero4());
    jobs[njob++] = job;
  }
  __syncthreads();  // every wave is done reading Qs / Ks (As, Ps do not alias them, WsT/UsT do later)
  for (int n = 0; n < njob; ++n) {
    const int which = jobs[n] / 10, t = jobs[n] % 10;
    int rb = 0;
    while ((rb + 1) * (rb + 2) / 2 <= t) ++rb;
    const int cb = t - rb * (rb + 1) / 2;
    const int j = cb * 16 + (l & 15);
    const float gj = sm.Gs[j];
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const int i = rb * 16 + 4 * (l >> 4) + i4;
      const float gi = sm.Gs[i];
      if (which == 0) {
        sm.As[i][j] = i > j ? sm.Bs[i] * __expf(gi - gj) * acc[n][i4] : 0.f;
      } else {
        sm.Ps[i][j] = f32_to_bf16(i >= j ? scale * __expf(gi - gj) * acc[n][i4] : 0.f);
      }
    }
  }
  // zero the strictly upper blocks of P (6 tiles of 16x16)
  for (int e = tid; e < 6 * 256; e += 64 * P1_WAVES) {
    const int t = e / 256, w = e % 256;
    const int rb = t < 3 ? 0 : (t < 5 ? 1 : 2);
    const int cb = t < 3 ? t + 1 : (t < 5 ? t - 1 : 3);
    sm.Ps[rb * 16 + w / 16][cb * 16 + w % 16] = 0;
  }
  __syncthreads();

  // 3a. diagonal 16x16 blocks of T by forward substitution: lane = 16 * block + column.
  if (wave == 0) {
    const int b = l >> 4, col = l & 15, base = b * 16;
    float t[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float s = (r == col) ? 1.f : 0.f;
#pragma unroll
      for (int jj = 0; jj < r; ++jj) s = fmaf(-sm.As[base + r][base + jj], t[jj], s);
      t[r] = s;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) sm.Ts[base + r][base + col] = t[r];
  }
  // zero the strictly upper blocks of T
  for (int e = tid; e < 6 * 256; e += 64 * P1_WAVES) {
    const int t = e / 256, w = e % 256;
    const int rb = t < 3 ? 0 : (t < 5 ? 1 : 2);
    const int cb = t < 3 ? t + 1 : (t < 5 ? t - 1 : 3);
    sm.Ts[rb * 16 + w / 16][cb * 16 + w % 16] = 0.f;
  }
  __syncthreads();

  // 3b. off-diagonal blocks, one block row at a time: T_ij = -T_ii sum_{m=j}^{i-1} A_im T_mj.
  for (int bi = 1; bi < 4; ++bi) {
    const int bj = wave;  // wave w computes block (bi, w) for w < bi
    if (bj < bi) {
      f32x4 y = zero4();
      for (int m = bj; m < bi; ++m) y = mm16_f32(&sm.As[bi * 16][m * 16], LDF, &sm.Ts[m * 16][bj * 16], LDF, y);
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) sm.Ys[wave][4 * (l >> 4) + i4][l & 15] = y[i4];
    }
    __syncthreads();
    if (bj < bi) {
      f32x4 z = mm16_f32(&sm.Ts[bi * 16][bi * 16], LDF, &sm.Ys[wave][0][0], 20, zero4());
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) sm.Ts[bi * 16 + 4 * (l >> 4) + i4][bj * 16 + (l & 15)] = -z[i4];
    }
    __syncthreads();
  }

  // 3c. TB = T diag(beta exp G), LB = (T - I) diag(beta), both bf16.
  for (int e = tid; e < CH * CH; e += 64 * P1_WAVES) {
    const int i = e / CH, j = e % CH;
    const float t = sm.Ts[i][j];
    sm.TBs[i][j] = f32_to_bf16(t * sm.Bs[j] * __expf(sm.Gs[j]));
    sm.LBs[i][j] = f32_to_bf16(i > j ? t * sm.Bs[j] : 0.f);
  }
  __syncthreads();

  // 4. W = TB K, Ub = beta V + LB V (32 tiles each); K^T to the workspace.
  {
    uint16_t* gW = reinterpret_cast<uint16_t*>(wsc + WS_W);
    float* gUT = reinterpret_cast<float*>(wsc + WS_UT);
    for (int job = wave; job < 64; job += P1_WAVES) {
      const int which = job >> 5, t = job & 31;
      const int rb = t >> 3, nb = t & 7;
      const int kend = rb < 2 ? 32 : 64;  // T and LB vanish above the block diagonal
      const int n = nb * 16 + (l & 15);
      const int i0 = rb * 16 + 4 * (l >> 4);
      if (which == 0) {
        f32x4 w = tile_mm(&sm.TBs[0][0], LDC, rb * 16, &sm.KsT[0][0], LDC, nb * 16, kend, zero4());
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          const uint16_t wb = f32_to_bf16(w[i4]);
          gW[(i0 + i4) * DK + n] = wb;
          sm.u.d.WsT[n][i0 + i4] = wb;
        }
      } else {
        f32x4 u = tile_mm(&sm.LBs[0][0], LDC, rb * 16, &sm.VsT[0][0], LDC, nb * 16, kend, zero4());
        float4 o;
        float* op = &o.x;
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          const int i = i0 + i4;
          const float val = fmaf(sm.Bs[i], bf16_to_f32(sm.VsT[n][i]), u[i4]);
          op[i4] = val;
          sm.u.d.UsT[n][i] = f32_to_bf16(val);
        }
        *reinterpret_cast<float4*>(gUT + n * CH + i0) = o;
      }
    }
    uint4* gKT = reinterpret_cast<uint4*>(wsc + WS_KT);
    for (int e = tid; e < DK * CH / 8; e += 64 * P1_WAVES) {
      const int n = e / (CH / 8), t8 = (e % (CH / 8)) * 8;
      gKT[e] = *reinterpret_cast<const uint4*>(&sm.KsT[n][t8]);
    }
  }
  __syncthreads();

  // 5. Qp = s exp(G) Q - P W, Ol = P Ub (32 tiles each).
  {
    uint16_t* gQp = reinterpret_cast<uint16_t*>(wsc + WS_QP);
    uint16_t* gOT = reinterpret_cast<uint16_t*>(wsc + WS_OT);
    for (int job = wave; job < 64; job += P1_WAVES) {
      const int which = job >> 5, t = job & 31;
      const int rb = t >> 3, nb = t & 7;
      const int kend = rb < 2 ? 32 : 64;
      const int n = nb * 16 + (l & 15);
      const int i0 = rb * 16 + 4 * (l >> 4);
      if (which == 0) {
        f32x4 pw = tile_mm(&sm.Ps[0][0], LDC, rb * 16, &sm.u.d.WsT[0][0], LDC, nb * 16, kend, zero4());
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          const int i = i0 + i4;
          float qv = 0.f;
          if (i < cr.len) qv = io<TIn>::load(q + ((size_t)(cr.t0 + i) * Hk + hk) * DK + n);
          gQp[i * DK + n] = f32_to_bf16(scale * __expf(sm.Gs[i]) * qv - pw[i4]);
        }
      } else {
        f32x4 ol = tile_mm(&sm.Ps[0][0], LDC, rb * 16, &sm.u.d.UsT[0][0], LDC, nb * 16, kend, zero4());
        uint2 w;
        w.x = (uint32_t)f32_to_bf16(ol[0]) | ((uint32_t)f32_to_bf16(ol[1]) << 16);
        w.y = (uint32_t)f32_to_bf16(ol[2]) | ((uint32_t)f32_to_bf16(ol[3]) << 16);
        *reinterpret_cast<uint2*>(gOT + n * CH + i0) = w;
      }
    }
  }
}

// ----------------------------------------------------------------------------------------------- phase 2

constexpr int P2_WAVES = 4;

template <typename TOut>
__global__ __launch_bounds__(64 * P2_WAVES) void chunk_state_kernel(
    const uint8_t* __restrict__ ws, const float* __restrict__ s_in, float* __restrict__ s_out,
    TOut* __restrict__ o, const int32_t* __restrict__ cu, int n_seqs, int n_chunks, int T, int Hv) {
  __shared__ uint16_t Ss[VB][LDQ];   // state slice (bf16), B operand of [Qp; W] S^T
  __shared__ uint16_t UhT[VB][LDC];  // decayed U^T, hi and lo parts: A operands of the state update
  __shared__ uint16_t UlT[VB][LDC];

  // XCD-aware order: the DV/VB workgroups of one (sequence, head) are `pairs` ids apart, so with
  // pairs % 8 == 0 they share an XCD and its L2 (they read the same chunk workspace).
  const int pairs = n_seqs * Hv;
  const int id = blockIdx.x;
  const int pair = id % pairs, vb = id / pairs;
  const int seq = pair / Hv, h = pair % Hv;
  const int l = lane_id(), wave = threadIdx.x >> 6;

  int bos, len, c0;
  if (cu != nullptr) {
    bos = cu[seq];
    len = cu[seq + 1] - bos;
    c0 = 0;
    for (int s = 0; s < seq; ++s) c0 += (cu[s + 1] - cu[s] + CH - 1) / CH;
  } else {
    bos = seq * T;
    len = T;
    c0 = seq * ((T + CH - 1) / CH);
  }
  // chunks past the workspace (a chunk table shorter than the sequences need) are not read
  const int nchunks = max(0, min((len + CH - 1) / CH, n_chunks - c0));

  // state slice in the D layout of the state update: rows j = 4*(l/16)+i, columns n = 32*wave + 16*tt + l%16
  f32x4 S[2];
  const size_t sbase = (((size_t)seq * Hv + h) * DV + vb * VB) * DK;
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int n = 32 * wave + 16 * tt + (l & 15);
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4)
      S[tt][i4] = s_in != nullptr ? s_in[sbase + (size_t)(4 * (l >> 4) + i4) * DK + n] : 0.f;
  }

  for (int ci = 0; ci < nchunks; ++ci) {
    const uint8_t* wsc = ws + ((size_t)(c0 + ci) * Hv + h) * WS_CHUNK;
    const uint16_t* gQp = reinterpret_cast<const uint16_t*>(wsc + WS_QP);
    const uint16_t* gW = reinterpret_cast<const uint16_t*>(wsc + WS_W);
    const uint16_t* gKT = reinterpret_cast<const uint16_t*>(wsc + WS_KT);
    const float* gUT = reinterpret_cast<const float*>(wsc + WS_UT);
    const uint16_t* gOT = reinterpret_cast<const uint16_t*>(wsc + WS_OT);
    const float* gG = reinterpret_cast<const float*>(wsc + WS_G);
    const int tlen = min(CH, len - ci * CH);

    // state slice -> LDS (bf16)
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int n = 32 * wave + 16 * tt + (l & 15);
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) Ss[4 * (l >> 4) + i4][n] = f32_to_bf16(S[tt][i4]);
    }
    __syncthreads();

    // [Qp; W] S^T for tokens 16*wave .. +15
    f32x4 xq = zero4(), xw = zero4();
#pragma unroll
    for (int k0 = 0; k0 < DK; k0 += 32) {
      const bf16x8 b = frag(&Ss[0][0], LDQ, 0, k0);
      xq = mfma(frag(gQp, DK, 16 * wave, k0), b, xq);
      xw = mfma(frag(gW, DK, 16 * wave, k0), b, xw);
    }
    const int j = l & 15;
    const int t0 = 16 * wave + 4 * (l >> 4);
    const float GL = gG[CH - 1];
    {
      // outputs O = Ol + Qp S^T
      const uint2 ow = *reinterpret_cast<const uint2*>(gOT + (vb * VB + j) * CH + t0);
      const float ol[4] = {__uint_as_float(ow.x << 16), __uint_as_float(ow.x & 0xffff0000u),
                           __uint_as_float(ow.y << 16), __uint_as_float(ow.y & 0xffff0000u)};
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const int t = t0 + i4;
        if (t < tlen) io<TOut>::store(o + ((size_t)(bos + ci * CH + t) * Hv + h) * DV + vb * VB + j, ol[i4] + xq[i4]);
      }
      // decayed corrected values -> LDS as hi + lo bf16
      const float4 ub = *reinterpret_cast<const float4*>(gUT + (vb * VB + j) * CH + t0);
      const float4 gt = *reinterpret_cast<const float4*>(gG + t0);
      const float us[4] = {(ub.x - xw[0]) * __expf(GL - gt.x), (ub.y - xw[1]) * __expf(GL - gt.y),
                           (ub.z - xw[2]) * __expf(GL - gt.z), (ub.w - xw[3]) * __expf(GL - gt.w)};
      uint32_t hi[4], lo[4];
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        hi[i4] = f32_to_bf16(us[i4]);
        lo[i4] = f32_to_bf16(us[i4] - bf16_to_f32((uint16_t)hi[i4]));
      }
      *reinterpret_cast<uint2*>(&UhT[j][t0]) = make_uint2(hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16));
      *reinterpret_cast<uint2*>(&UlT[j][t0]) = make_uint2(lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16));
    }
    __syncthreads();

    // S = exp(G_L) S + (decayed U)^T K for columns 32*wave .. +31
    const float dec = __expf(GL);
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      f32x4 acc = S[tt] * dec;
      const int n0 = 32 * wave + 16 * tt;
#pragma unroll
      for (int k0 = 0; k0 < CH; k0 += 32) {
        const bf16x8 kb = frag(gKT, CH, n0, k0);
        acc = mfma(frag(&UhT[0][0], LDC, 0, k0), kb, acc);
        acc = mfma(frag(&UlT[0][0], LDC, 0, k0), kb, acc);
      }
      S[tt] = acc;
    }
    __syncthreads();  // Ss / UhT / UlT are rewritten by the next chunk
  }

  if (s_out != nullptr) {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int n = 32 * wave + 16 * tt + (l & 15);
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) s_out[sbase + (size_t)(4 * (l >> 4) + i4) * DK + n] = S[tt][i4];
    }
  }
}

template <typename TIn, typename TG>
void launch_prep(bool gate, int nchunks, int Hk, int Hv, const void* q, const void* k, const void* v, const void* g,
                 const void* beta, const float* A_log, const float* dt_bias, const int32_t* cu,
                 const int32_t* chunk_idx, int n_seqs, int T, float scale, uint8_t* ws, hipStream_t stream) {
  dim3 grid(nchunks, Hv);
  if (gate)
    hipLaunchKernelGGL((chunk_prep_kernel<TIn, TG, true>), grid, dim3(64 * P1_WAVES), 0, stream, (const TIn*)q,
                       (const TIn*)k, (const TIn*)v, (const TG*)g, (const TG*)beta, A_log, dt_bias, cu, chunk_idx,
                       n_seqs, T, Hk, Hv, scale, ws);
  else
    hipLaunchKernelGGL((chunk_prep_kernel<TIn, TG, false>), grid, dim3(64 * P1_WAVES), 0, stream, (const TIn*)q,
                       (const TIn*)k, (const TIn*)v, (const TG*)g, (const TG*)beta, A_log, dt_bias, cu, chunk_idx,
                       n_seqs, T, Hk, Hv, scale, ws);
}

}  // namespace
}  // namespace zgdn

extern "C" size_t zgdn_chunk_workspace_size(int n_chunks, int Hv) {
  return (size_t)(n_chunks > 0 ? n_chunks : 0) * (size_t)(Hv > 0 ? Hv : 0) * zgdn::WS_CHUNK;
}

extern "C" int zgdn_chunk_fwd(const void* q, const void* k, const void* v, int qkv_dtype, const void* g,
                              const void* beta, int gb_dtype, const float* A_log, const float* dt_bias,
                              const float* initial_state, float* final_state, void* o,
                              const int32_t* cu_seqlens, const int32_t* chunk_indices, int n_seqs, int n_chunks,
                              int B, int T, int Hk, int Hv, int K, int V, float scale, void* workspace,
                              size_t workspace_bytes, void* stream) {
  using namespace zgdn;
  const char* fn = "zgdn_chunk_fwd";
  if (!q || !k || !v || !g || !beta || !o || !workspace) return fail(ZGDN_EINVAL, "%s: null pointer", fn);
  if (K != DK || V != DV) return fail(ZGDN_EUNSUPPORTED, "%s: K=%d V=%d (supported: 128, 128)", fn, K, V);
  if (qkv_dtype != ZGDN_BF16) return fail(ZGDN_EUNSUPPORTED, "%s: q/k/v must be bf16", fn);
  if (gb_dtype != ZGDN_F32 && gb_dtype != ZGDN_BF16) return fail(ZGDN_EINVAL, "%s: dtype code %d", fn, gb_dtype);
  if (B < 1 || T < 0 || Hk < 1 || Hv < 1 || Hv % Hk)
    return fail(ZGDN_EINVAL, "%s: bad sizes B=%d T=%d Hk=%d Hv=%d", fn, B, T, Hk, Hv);
  if ((A_log == nullptr) != (dt_bias == nullptr))
    return fail(ZGDN_EINVAL, "%s: A_log and dt_bias go together", fn);
  int N = B;
  if (cu_seqlens != nullptr) {
    if (B != 1 || chunk_indices == nullptr || n_seqs < 1)
      return fail(ZGDN_EINVAL, "%s: packed sequences need B == 1, chunk_indices and n_seqs >= 1", fn);
    N = n_seqs;
  } else {
    n_chunks = B * ((T + CH - 1) / CH);
  }
  if (n_chunks < 0) return fail(ZGDN_EINVAL, "%s: n_chunks=%d", fn, n_chunks);
  if (workspace_bytes < zgdn_chunk_workspace_size(n_chunks, Hv))
    return fail(ZGDN_EINVAL, "%s: workspace of %zu bytes, need %zu", fn, workspace_bytes,
                zgdn_chunk_workspace_size(n_chunks, Hv));
  hipStream_t s = (hipStream_t)stream;
  uint8_t* ws = (uint8_t*)workspace;
  const bool gate = A_log != nullptr;
  if (n_chunks > 0) {
    if (gb_dtype == ZGDN_F32)
      launch_prep<bf16, float>(gate, n_chunks, Hk, Hv, q, k, v, g, beta, A_log, dt_bias, cu_seqlens, chunk_indices,
                               N, T, scale, ws, s);
    else
      launch_prep<bf16, bf16>(gate, n_chunks, Hk, Hv, q, k, v, g, beta, A_log, dt_bias, cu_seqlens, chunk_indices,
                              N, T, scale, ws, s);
  }
  dim3 grid2(N * Hv * (DV / VB));
  hipLaunchKernelGGL((chunk_state_kernel<bf16>), grid2, dim3(64 * P2_WAVES), 0, s, ws, initial_state, final_state,
                     (bf16*)o, cu_seqlens, N, n_chunks, T, Hv);
  return check_launch(fn);
}
