// Chunked (WY / UT form) gated delta rule prefill on bf16 MFMA, 64-token chunks, dk = dv = 128.
//
// Per chunk of L <= 64 tokens and value head h, with in-chunk cumulative log decay G (G_i = g_1+..+g_i), start
// state S0 [V, K] (value-major) and scale s (the chunked statement of the recurrence):
//   A  = strictly-lower( beta_i exp(G_i - G_j) k_i.k_j )           T = (I + A)^-1   (unit lower triangular)
//   W  = T diag(beta exp(G)) K                                      [L x K]
//   Ub = diag(beta) V + (T - I) diag(beta) V                        [L x V]   (diagonal exact in fp32)
//   P  = s * lower-incl( exp(G_i - G_j) q_i.k_j )                   [L x L]
//   U  = Ub - W S0^T                                                (the corrected values)
//   O  = s diag(exp(G)) Q S0^T + P U  =  Q' S0^T + Ob,   Q' = s diag(exp(G)) Q - P W,   Ob = P Ub
//   S  = exp(G_L) S0 + U'^T K,   U' = diag(exp(G_L - G)) U = Ub' - W' S0^T  (Ub', W' the rows of Ub, W scaled)
// Phase 1 (chunk_prep_kernel, one item per chunk x head, all independent) forms W', Q', K^T, Ub', Ob and
// G_L into a workspace. Phase 2 (chunk_state_kernel, one workgroup per sequence x head x 16 value rows) walks
// the chunks in order keeping its 16 x 128 slice of the fp32 state in registers: one MFMA pass over [W'; Q']
// gives U' and the outputs, a second the state update. Only the state pass is sequential, so the workspace is
// stored in MFMA fragment order: every phase-2 operand load is one contiguous 1 KiB per wave (rows read
// straight from row-major matrices cost about 2.3x as much per byte on CDNA), and the next chunk's loads are
// issued in three groups spread over the current chunk so they overlap its MFMA and LDS work.
// Numerics: MFMA operands are bf16 with fp32 accumulation; U' enters the state update as a hi + lo bf16 pair
// (two MFMAs) and the diagonal of T diag(beta) is applied in fp32, which keeps the fp32 state within ~1e-4 of
// the exact recurrence; the output path (Q', Ob, S in bf16) stays within ~1e-3 of |o|.
//
// With the q/k L2-norm fused in (lm.py:570-571), q_t = rq_t cq_t and k_t = rk_t ck_t where cq, ck are the
// raw (exactly bf16) rows and rq, rk = rsqrt(sum c^2 + 1e-6) are fp32: every factor r is folded into the
// fp32 side of the products (A, P, the columns of T diag(beta exp(G) rk), Fq_t = s exp(G_t) rq_t and
// Fk_t = exp(G_L - G_t) rk_t), so the normalised q, k are never rounded to bf16.
//
// MFMA used: v_mfma_f32_16x16x32_bf16 (A: row lane%16, k 8*(lane/16)+0..7; B: column lane%16, same k;
// D: row 4*(lane/16)+i, column lane%16) and v_mfma_f32_16x16x4_f32 (A[lane%16][lane/16], B[lane/16][lane%16])
// for the fp32 block inverse. The contraction index of the [W'; Q'] S^T pass is taken in a permuted key order
// (kappa below) so that two 16 x 16 D tiles of W'^T computed in phase 1 are directly one A fragment.
#include <type_traits>
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <mutex>

#include "gdn_common.h"

namespace zgdn {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int CH = 64;    // chunk length
constexpr int DK = 128;   // key dim
constexpr int DV = 128;   // value dim
constexpr int VB = 16;    // value rows per phase-2 workgroup (DV / VB = 8 workgroups per sequence x head)

// x = hi + lo for a pair of floats: hi their bf16 rounding, lo the bf16 rounding of what is left (together
// about 16 significant bits)
__device__ __forceinline__ void split2(float a, float b, uint32_t& hi, uint32_t& lo) {
  hi = pack_bf16x2(a, b);
  lo = pack_bf16x2(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xffff0000u));
}

constexpr int LDC = CH + 8;  // padded LDS row (bf16) of a 64-wide matrix
constexpr int LDF = CH + 4;  // padded LDS row (fp32) of a 64-wide matrix

// Workspace of one chunk x head (bytes), every block in the register order of the phase-2 wave that reads it.
// Token tile tb = 16 tokens, value block vb = 16 value rows, k-step kk = 32 keys; lane l:
//   W'  [tb][kk][l] 8 bf16: W'[16 tb + l%16][kappa(kk, l, 0..7)]        (A fragments, U role)
//   Q'  [tb][kk][l] 8 bf16: Q'[16 tb + l%16][kappa(kk, l, 0..7)]        (A fragments, O role)
//   K^T [w][kk][l]  8 bf16: k[32 kk + 8 (l/16) + 0..7][16 w + l%16]     (B fragments of the state update)
//   Ub' [vb][tb][l] 4 f32 : Ub'[16 tb + 4 (l/16) + i][16 vb + l%16]     (D tiles)
//   Ob  [vb][tb][l] 4 bf16: Ob[16 tb + 4 (l/16) + i][16 vb + l%16]      (D tiles)
//   G_L, then padding to a 256-byte multiple.
// kappa(kk, l, i) = 32 kk + 4 (l/16) + i for i < 4 and 32 kk + 16 + 4 (l/16) + i - 4 for i >= 4.
// (Phase 1 keeps the k and v rows row-major in LDS and reads the K^T / V^T operands with transposing LDS
// reads.)
constexpr size_t WS_WP = 0;
constexpr size_t WS_QP = WS_WP + CH * DK * 2;
constexpr size_t WS_KT = WS_QP + CH * DK * 2;
constexpr size_t WS_UB = WS_KT + DK * CH * 2;
constexpr size_t WS_OB = WS_UB + CH * DV * 4;
constexpr size_t WS_GL = WS_OB + CH * DV * 2;
constexpr size_t WS_CHUNK = WS_GL + 256;  // 98,560 bytes

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

// Two D tiles (keys 32 kk + 0..15 and 32 kk + 16..31, one token column per lane) as one bf16 A fragment in
// the kappa key order.
__device__ __forceinline__ uint4 kappa_frag(f32x4 d0, f32x4 d1) {
  return make_uint4(pack_bf16x2(d0[0], d0[1]), pack_bf16x2(d0[2], d0[3]), pack_bf16x2(d1[0], d1[1]),
                    pack_bf16x2(d1[2], d1[3]));
}


// ----------------------------------------------------------------------------------------------- phase 1

constexpr int P1_WAVES = 8;
constexpr int P1_THREADS = 64 * P1_WAVES;
constexpr int P1_WGS_PER_CU = 2;
constexpr int P1_WAVES_PER_SIMD = P1_WGS_PER_CU * P1_WAVES / 4;  // caps the registers per wave at 512 / 4

typedef short short4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Lower-triangle tile t (0..9) of a 4x4 block grid -> (row block, column block), row-major order.
__device__ __forceinline__ void lower_tile(int t, int& rb, int& cb) {
  rb = t < 1 ? 0 : (t < 3 ? 1 : (t < 6 ? 2 : 3));
  cb = t - rb * (rb + 1) / 2;
}

// Contraction length over tokens for token tile tb of a lower-triangular left operand.
__device__ __forceinline__ int tri_kend(int tb) { return tb < 2 ? 32 : 64; }


// ----------------------------------------------------------------------------------------------- phase 1
//
// One item = one (chunk, value head): W', Q', K^T, Ub', Ob and G_L of the chunk into its workspace. Persistent
// workgroups of 8 waves, two per CU (75,776 bytes of LDS each), loop over items. The item is laid out for few
// VALU instructions and a short dependent chain:
// * every LDS access is a per-lane offset formed once plus a compile-time or wave-uniform part: the XOR
//   swizzles (16-byte chunk c of row r at c ^ (r % 16) for 256-byte rows, c ^ ((r / 2) % 8) for 128-byte rows,
//   which keeps 16-row fragment reads free of bank conflicts without padding) are arranged so that a tile's or
//   k-step's part is one XOR or an immediate on the lane's offset;
// * a D tile is stored transposed (row n of X^T holds the tile's 4 rows of column n: one 16-byte fp32 or 8-byte
//   bf16 write a lane), and its consumers read X's row fragments with transposing reads (ds_read_b64_tr_b16:
//   within 16 lanes, lane s names row k0 + s/4, columns c0 + 4 (s%4) .. + 3, and lane i receives column c0 + i
//   of the 4 rows) or take X^T's rows: A^T, P^T, T^T, (diag(Fk) T diag(Bk))^T, ((T - I) diag(beta))^T, R^T, Ub^T;
// * the rows are read with buffer loads (a scalar base per item; rows past the chunk end fall outside the
//   buffer range and read zero), the next item's rows in flight while the current item computes;
// * the diagonal 16x16 blocks of T = (I + A)^-1 are inverted by one wave by right-looking substitution from rows
//   of A^T (column c of a block per lane: once t_m is final every later row's partial sum takes one FMA, so the
//   dependent chain is one FMA a row, not a row's dot product) while the other waves scale and store the other
//   tiles; the off-diagonal blocks follow in three levels of 16x16 fp32 block products:
//   N_ij = T_ii A_ij; T_10, T_21, T_32 = -N_10 T_00, -N_21 T_11, -N_32 T_22 and the pair products N_21 N_10,
//   N_32 N_20, N_32 N_21; then T_20 = (N_21 N_10 - N_20) T_00, T_31 = (N_32 N_21 - N_31) T_11 and
//   T_30 = (N_32 N_20 - N_30) T_00 + (N_32 N_21 - N_31) T_10;
// * barriers wait for LDS traffic only: the workspace stores and the next item's loads stay in flight.
// (An earlier form of this item recomputed its swizzled addresses per element and took the diagonal blocks by
// a row-by-row dot-product substitution: 10.1-10.9k VALU instructions an item against 5.3k, 38.5 against
// 30.7 us for the 1,024 items of a 4096-token, 16-head prefill.)

// byte offsets in the item's LDS block
constexpr int PS_Q = 0;            // raw q rows [64][128] bf16 (256-byte rows)        } one 32 KiB region,
constexpr int PS_AT = 0;           // A^T, then N^T in its blocks, fp32 [64][64]        } reused by phase
constexpr int PS_TT = 16384;       // T^T fp32 (logical blocks (0, 1..3): pair products)
constexpr int PS_TBF = 0;          // (diag(Fk) T diag(Bk))^T bf16 [64][64] (128-byte rows)
constexpr int PS_TBT = 8192;       // (T diag(Bk))^T
constexpr int PS_LB = 16384;       // ((T - I) diag(beta))^T
constexpr int PS_RT = 24576;       // R^T
constexpr int PS_UBT = 0;          // Ub^T bf16 [128][64]
constexpr int PS_K = 32768;        // k rows [64][128] bf16
constexpr int PS_V = 49152;        // v rows
constexpr int PS_PT = 65536;       // P^T bf16 [64][64]; the blocks of zeros above P's diagonal blocks set once
constexpr int PS_F = 73728;        // per-token factors: 8 x 64 floats
constexpr int PSF_G = 0, PSF_B = 256, PSF_H = 512, PSF_UA = 768, PSF_UP = 1024, PSF_BK = 1280, PSF_FQ = 1536,
              PSF_FK = 1792;
constexpr int PS_BYTES = PS_F + 2048;  // 75,776
struct alignas(16) PrepShared {
  uint8_t b[PS_BYTES];
};

template <typename T>
__device__ __forceinline__ T lds_at(const uint8_t* base, int off) {
  return *reinterpret_cast<const T*>(base + off);
}
template <typename T>
__device__ __forceinline__ void lds_put(uint8_t* base, int off, T v) {
  *reinterpret_cast<T*>(base + off) = v;
}
__device__ __forceinline__ uint2 lds_tr(const uint8_t* base, int off) {
  return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                       (__attribute__((address_space(3))) short4_t*)(base + off)));
}

// Per-lane LDS offsets, formed once per workgroup (lane l, m = l % 16, g = l / 16).
struct PrepLane {
  int f16[4];    // row fragment (rows r0 + m, k = 32 kk + 8 g ..) of a 256-byte-row matrix: + 256 r0
  int f8[2];     // the same for 128-byte rows: + 128 r0
  int t16, t16h;  // transposing-read fragment of a 256-byte-row matrix: (t ^ 2 r0) + 8192 kk
  int t8, t8h;   // the same for 128-byte rows: (t ^ 2 r0) + 4096 kk
  int w32;       // transposed D-tile store, fp32 256-byte rows: (w32 ^ 64 ri) + 4096 rj
  int w16;       // transposed D-tile store, bf16 128-byte rows: (w16 ^ 32 ri) + 2048 rj
  int rA, rB;    // fp32 block operands of the 16x16x4 products (see mm_t)
  int dv;        // exact-diagonal read of v rows (4 rows i0 .., 4 columns): (dv ^ 32 vb) + 4096 tb
  __device__ __forceinline__ explicit PrepLane(int l) {
    const int m = l & 15, g = l >> 4, s = m;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) f16[kk] = m * 256 + (((4 * kk + g) ^ m) << 4);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) f8[kk] = m * 128 + (((4 * kk + g) ^ (m >> 1)) << 4);
    const int y16 = 8 * (g & 1) + (s >> 2);
    t16 = (8 * g + (s >> 2)) * 256 + ((((s & 3) >> 1) ^ y16) << 4) + 8 * (s & 1);
    t16h = (t16 + 1024) ^ 64;
    const int y8 = 4 * (g & 1) + (s >> 3);
    t8 = (8 * g + (s >> 2)) * 128 + ((((s & 3) >> 1) ^ y8) << 4) + 8 * (s & 1);
    t8h = (t8 + 512) ^ 32;
    w32 = m * 256 + ((g ^ m) << 4);
    w16 = m * 128 + ((((g >> 1) ^ (m >> 1))) << 4) + 8 * (g & 1);
    rA = g * 256 + ((((m >> 2) ^ g)) << 4) + (m & 3) * 4;
    rB = m * 256 + (m << 4) + g * 4;
    dv = (4 * g + (m >> 2)) * 256 + ((((m & 3) >> 1) ^ (4 * g + (m >> 2))) << 4) + 8 * (m & 1);
  }
};

// Row fragment (rows r0 + lane%16, k-step kk) of a row-major swizzled matrix at byte `mat`.
__device__ __forceinline__ bf16x8 pfrag16(const uint8_t* lb, int mat, int r0, int kk, const PrepLane& L) {
  return lds_at<bf16x8>(lb, mat + 256 * r0 + L.f16[kk]);
}
__device__ __forceinline__ bf16x8 pfrag8(const uint8_t* lb, int mat, int r0, int kk, const PrepLane& L) {
  return lds_at<bf16x8>(lb, mat + 128 * r0 + L.f8[kk]);
}
// Row fragment of M (rows r0 + lane%16 of M, k-step kk) read from M^T stored row-major (transposing reads):
// 256-byte rows of M^T (M^T has 64 rows: k up to 64, columns up to 128) and 128-byte rows (64 columns).
__device__ __forceinline__ bf16x8 pfragT16(const uint8_t* lb, int mat, int r0, int kk, const PrepLane& L) {
  const uint2 a = lds_tr(lb, mat + 8192 * kk + (L.t16 ^ (2 * r0)));
  const uint2 b = lds_tr(lb, mat + 8192 * kk + (L.t16h ^ (2 * r0)));
  return __builtin_bit_cast(bf16x8, make_uint4(a.x, a.y, b.x, b.y));
}
__device__ __forceinline__ bf16x8 pfragT8(const uint8_t* lb, int mat, int r0, int kk, const PrepLane& L) {
  const uint2 a = lds_tr(lb, mat + 4096 * kk + (L.t8 ^ (2 * r0)));
  const uint2 b = lds_tr(lb, mat + 4096 * kk + (L.t8h ^ (2 * r0)));
  return __builtin_bit_cast(bf16x8, make_uint4(a.x, a.y, b.x, b.y));
}
// D tile (rows 16 ri + 4 (lane/16) + i, column 16 rj + lane%16) stored transposed: fp32 into 256-byte rows,
// bf16 (4 values, 8 bytes) into 128-byte rows.
__device__ __forceinline__ void put_t32(uint8_t* lb, int mat, int ri, int rj, const PrepLane& L, f32x4 d) {
  lds_put<f32x4>(lb, mat + 4096 * rj + (L.w32 ^ (64 * ri)), d);
}
__device__ __forceinline__ void put_t16(uint8_t* lb, int mat, int ri, int rj, const PrepLane& L, f32x4 d) {
  lds_put<uint2>(lb, mat + 2048 * rj + (L.w16 ^ (32 * ri)), make_uint2(pack_bf16x2(d[0], d[1]), pack_bf16x2(d[2], d[3])));
}
// acc += X[bi][bj] . Y[ci][cj] for 16x16 fp32 blocks of matrices stored transposed (X^T, Y^T row-major,
// 256-byte rows, fp32 swizzle), on v_mfma_f32_16x16x4_f32: A element X[16 bi + m][16 bj + 4 s + g] at row
// 16 bj + 4 s + g, column 16 bi + m of X^T; B element Y[16 ci + 4 s + g][16 cj + m] at row 16 cj + m, column
// 16 ci + 4 s + g of Y^T. `sub` (nonnegative mat2): A element X - X2[b2i][b2j].
__device__ __forceinline__ float lA(const uint8_t* lb, int mat, int bi, int bj, int s, const PrepLane& L) {
  return lds_at<float>(lb, mat + 4096 * bj + 1024 * s + ((bi ^ s) << 6) + L.rA);
}
__device__ __forceinline__ float lB(const uint8_t* lb, int mat, int ci, int cj, int s, const PrepLane& L) {
  return lds_at<float>(lb, mat + 4096 * cj + (L.rB ^ ((4 * ci ^ s) << 4)));
}
__device__ __forceinline__ f32x4 mm_t(const uint8_t* lb, int xm, int bi, int bj, int ym, int ci, int cj,
                                      const PrepLane& L, f32x4 acc) {
#pragma unroll
  for (int s = 0; s < 4; ++s)
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(lA(lb, xm, bi, bj, s, L), lB(lb, ym, ci, cj, s, L), acc, 0, 0, 0);
  return acc;
}
__device__ __forceinline__ f32x4 mm_t_diff(const uint8_t* lb, int xm, int bi, int bj, int x2m, int b2i, int b2j,
                                           int ym, int ci, int cj, const PrepLane& L, f32x4 acc) {
#pragma unroll
  for (int s = 0; s < 4; ++s)
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(lA(lb, xm, bi, bj, s, L) - lA(lb, x2m, b2i, b2j, s, L),
                                                lB(lb, ym, ci, cj, s, L), acc, 0, 0, 0);
  return acc;
}

// Buffer resource over rows [t0, t0 + len) of a row-major bf16 array (row stride `ld` elements), starting at
// column `col`: a row's byte at (row - t0) * 2 ld + 2 (c - col); rows from len on read zero.
__device__ __forceinline__ Rsrc rows_rsrc(const uint16_t* p, long t0, long ld, int col, int len) {
  return raw_rsrc(p + t0 * ld + col, (uint32_t)(len > 0 ? len : 0) * (uint32_t)ld * 2u);
}

struct RowRegs {
  uint4 q0, q1, k0, k1, v0, v1;
};

// Where a phase-1 item's rows lie: chunk c (its token range cr), value head h and key head hk.
struct ItemAt {
  int c, h, hk;
  ChunkRange cr;
};
__device__ __forceinline__ ItemAt item_at(int item, const int32_t* cu, const int32_t* chunk_idx, int n_seqs, int T,
                                          int Hk, int Hv) {
  ItemAt a;
  a.c = item / Hv;
  a.h = item % Hv;
  a.hk = a.h / (Hv / Hk);
  a.cr = chunk_range(a.c, cu, chunk_idx, T, n_seqs);
  return a;
}

// The items item0, item0 + stride, ... of a persistent workgroup with their positions carried from one to the
// next by additions (item = c Hv + h, and for B x T batches c = b nt + j with nt chunks a row): the integer
// divisions of item_at, each a dozen vector instructions (no scalar divide), are taken once per workgroup.
struct ItemWalk {
  int item, c, h, b, j;
  int stride, dc, dh, db, dj, Hv, nt, grp;
  uint32_t mg;  // ceil(2^32 / grp): h / grp = umulhi(h, mg), exact for h, grp < 2^16
  __device__ __forceinline__ ItemWalk(int item0, int stride_, int Hv_, int Hk, int T)
      : item(item0), stride(stride_), Hv(Hv_) {
    c = item0 / Hv;
    h = item0 % Hv;
    dc = stride / Hv;
    dh = stride % Hv;
    nt = max(1, (T + CH - 1) / CH);
    b = c / nt;
    j = c % nt;
    db = dc / nt;
    dj = dc % nt;
    grp = Hv / Hk;
    mg = grp > 1 ? 0xffffffffu / (uint32_t)grp + 1u : 0u;
  }
  __device__ __forceinline__ void advance() {
    item += stride;
    h += dh;
    const int carry = h >= Hv ? 1 : 0;
    h -= carry * Hv;
    c += dc + carry;
    j += dj + carry;
    b += db;
    if (j >= nt) {
      j -= nt;
      ++b;
    }
  }
  __device__ __forceinline__ ItemAt at(const int32_t* cu, const int32_t* chunk_idx, int n_seqs, int T) const {
    ItemAt a;
    a.c = c;
    a.h = h;
    a.hk = grp > 1 ? (int)__umulhi((uint32_t)h, mg) : h;
    if (cu != nullptr) {
      a.cr = chunk_range(c, cu, chunk_idx, T, n_seqs);
    } else {
      a.cr.t0 = b * T + j * CH;
      a.cr.len = min(CH, T - j * CH);
    }
    return a;
  }
};

// The chunk's rows of q, k, v for thread (rr, c8): rows rr and rr + 32 (W = 8 waves) or row rr (W = 16),
// columns c8 .. c8 + 7 (zeros past the chunk end).
template <int W>
__device__ __forceinline__ void load_rows(RowRegs& R, const ItemAt& it, const uint16_t* q, const uint16_t* k,
                                          const uint16_t* v, const RowStrides& rs, uint32_t oq, uint32_t ok,
                                          uint32_t ov) {
  const ChunkRange cr = it.cr;
  const int h = it.h, hk = it.hk;
  const Rsrc rq = rows_rsrc(q, cr.t0, rs.q, hk * DK, cr.len), rk = rows_rsrc(k, cr.t0, rs.k, hk * DK, cr.len);
  const Rsrc rv = rows_rsrc(v, cr.t0, rs.v, h * DV, cr.len);
  R.q0 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rq, oq, 0, 0));
  R.k0 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, ok, 0, 0));
  R.v0 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, ov, 0, 0));
  if constexpr (W == 8) {
    R.q1 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rq, oq + 64u * (uint32_t)rs.q, 0, 0));
    R.k1 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, ok + 64u * (uint32_t)rs.k, 0, 0));
    R.v1 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, ov + 64u * (uint32_t)rs.v, 0, 0));
  }
}

// Once per workgroup: the blocks of P^T that stay zero (P's blocks above its diagonal blocks).
__device__ __forceinline__ void prep_init(uint8_t* lb) {
  // P^T physical blocks (pr, pc) with pr > pc: (1,0), (2,0), (2,1), (3,0), (3,1), (3,2); 512 bytes each
  for (int e = threadIdx.x; e < 6 * 32; e += blockDim.x) {
    const int t = e >> 5, w = e & 31;
    const int pr = t < 1 ? 1 : (t < 3 ? 2 : 3), pc = t - pr * (pr - 1) / 2;
    const int row = 16 * pr + (w >> 1), c8 = 16 * pc + 8 * (w & 1);  // 8 bf16 of a row
    lds_put<uint4>(lb, PS_PT + row * 128 + ((((c8 >> 3) ^ ((row >> 1) & 7))) << 4), make_uint4(0, 0, 0, 0));
  }
}

// Workgroup barrier over the item's LDS traffic only: it waits for this wave's LDS accesses, not for its
// global loads and stores (the next item's rows, the workspace stores stay in flight across it; nothing of the
// workspace is read back by the item).
__device__ __forceinline__ void item_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// One phase-1 item (`it`). `R` holds the item's rows (loaded by the caller); with `has_next`, the rows of item
// `nx` are loaded into R while this one computes. QL: the raw q of the Q' step is taken from the q rows in LDS
// (held in registers from step 2 on; no second read of q from memory), else read again from memory before step
// 6 (fewer registers held: the overlapped kernel's budget). W: the workgroup's waves, 8 (two workgroups a CU) or
// 16 (one item a CU when the items are few: the phases spread over twice the waves, the item's latency
// shorter). Ends with a workgroup barrier.
template <typename TG, bool GATE, bool QL, int W>
__device__ __forceinline__ void prep_item(uint8_t* lb, const ItemAt& it, RowRegs& R, bool has_next, const ItemAt& nx,
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const TG* __restrict__ g, const TG* __restrict__ beta, const float* __restrict__ A_log,
    const float* __restrict__ dt_bias, int Hv, float scale, int qk_l2norm, const RowStrides& rs,
    uint8_t* __restrict__ ws, const PrepLane& L0, int rowoff, uint32_t oq, uint32_t ok, uint32_t ov) {
  // the lane offsets pass through an empty asm per item: the compiler then forms the addresses derived from
  // them inside the item (most fold into instruction offsets) instead of hoisting every one of them out of the
  // item loop, where they would not fit the registers
  PrepLane L = L0;
#pragma unroll
  for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(L.f16[i]));
  asm volatile("" : "+v"(L.f8[0]), "+v"(L.f8[1]), "+v"(L.t16), "+v"(L.t16h), "+v"(L.t8), "+v"(L.t8h));
  asm volatile("" : "+v"(L.w32), "+v"(L.w16), "+v"(L.rA), "+v"(L.rB), "+v"(L.dv), "+v"(rowoff));
  int tid = threadIdx.x;  // (opaque per item as well, for the values derived from it)
  asm volatile("" : "+v"(tid));
  const int l = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int m = l & 15, gq = l >> 4;
  const int c = it.c, h = it.h, hk = it.hk;
  const ChunkRange cr = it.cr;
  uint8_t* wsc = ws + ((size_t)c * Hv + h) * WS_CHUNK;
  float* F = reinterpret_cast<float*>(lb + PS_F);
  static_assert(W == 8 || W == 16, "8 or 16 waves an item");
  constexpr int NJ16 = 16 / W;                 // a wave's jobs of 16
  constexpr int NJ = (16 + W - 2) / (W - 1);   // a wave's jobs of the 16 off-diagonal K K^T / Q K^T tiles
  constexpr int TBN = 4 * 8 / W;               // token tiles of a wave's value block (steps 7, 8)

  // gate inputs (wave 7), issued before the row stores
  float gi = 0.f, bi = 0.f, alog = 0.f, dtb = 0.f;
  if (wave == W - 1 && l < cr.len) {
    const size_t gh = (size_t)(cr.t0 + l) * rs.gb + h;
    gi = io<TG>::load(g + gh);
    bi = io<TG>::load(beta + gh);
    if constexpr (GATE) {
      alog = A_log[h];
      dtb = dt_bias[h];
    }
  }
  // 1. rows -> LDS; the next item's rows into the registers
  lds_put<uint4>(lb, PS_Q + rowoff, R.q0);
  lds_put<uint4>(lb, PS_K + rowoff, R.k0);
  lds_put<uint4>(lb, PS_V + rowoff, R.v0);
  if constexpr (W == 8) {
    lds_put<uint4>(lb, PS_Q + rowoff + 8192, R.q1);
    lds_put<uint4>(lb, PS_K + rowoff + 8192, R.k1);
    lds_put<uint4>(lb, PS_V + rowoff + 8192, R.v1);
  }
  if (has_next) load_rows<W>(R, nx, q, k, v, rs, oq, ok, ov);
  if (wave == W - 1) {
    if (l < cr.len) {
      if constexpr (GATE) gi = -__expf(alog) * softplus(gi + dtb);
      if (rs.beta_sigmoid) bi = sigmoid(bi);
    }
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const float o = __shfl_up(gi, d);
      if (l >= d) gi += o;
    }
    F[(PSF_G >> 2) + l] = gi;
    F[(PSF_B >> 2) + l] = bi;
  }
  item_barrier();

  // 2. factors (threads 0-127: q rows, then k rows) and the K K^T / Q K^T tiles. Wave 0 takes the 4 diagonal
  // K K^T tiles (it inverts those blocks next); waves 1-7 take the other 16 tiles (jobs j: 0-5 the K K^T tiles
  // below the diagonal blocks, 6-15 the Q K^T tiles on and below them).
  if (tid < 2 * CH) {
    const int r = tid & (CH - 1);
    const int mat = tid < CH ? PS_Q : PS_K;
    float rf = 1.f;
    if (qk_l2norm) {
      float ss = 0.f;
      const int base = mat + r * 256 + ((r & 15) << 4);
#pragma unroll
      for (int cc = 0; cc < 16; ++cc) {  // physical chunk cc ^ (r % 16): every lane of 16 on its own banks
        const uint4 w4 = lds_at<uint4>(lb, base ^ (cc << 4));
        const uint32_t u[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bf16x2 x = __builtin_bit_cast(bf16x2, u[i]);
          ss = __builtin_amdgcn_fdot2_f32_bf16(x, x, ss, false);
        }
      }
      rf = rsqrtf(ss + 1e-6f);
    }
    const float gr = F[(PSF_G >> 2) + r], g2 = gr * 1.44269504088896341f;  // G in log2 units
    if (tid < CH) {
      F[(PSF_UP >> 2) + r] = g2 + __builtin_amdgcn_logf(scale * rf);
      F[(PSF_FQ >> 2) + r] = scale * __expf(gr) * rf;
    } else {
      const float br = F[(PSF_B >> 2) + r];
      F[(PSF_H >> 2) + r] = g2 - __builtin_amdgcn_logf(rf);
      F[(PSF_UA >> 2) + r] = g2 + __builtin_amdgcn_logf(br * rf);  // (-inf for beta = 0: those rows of A are 0)
      F[(PSF_FK >> 2) + r] = __expf(F[(PSF_G >> 2) + CH - 1] - gr) * rf;
      F[(PSF_BK >> 2) + r] = br * __expf(gr) * rf;
    }
  }
  // raw q of this wave's Q' jobs (step 8): token 16 tb + m, columns 32 kq + 4 gq .. + 3 and 16 further; with QL
  // from the q rows, before A^T overwrites them (rows past the chunk end hold zeros)
  uint2 cq[NJ16][2];
  if constexpr (QL) {
#pragma unroll
    for (int n = 0; n < NJ16; ++n) {
      const int job = wave + W * n, tb = job >> 2, kq = job & 3;
      const int tok = 16 * tb + m, cc = 4 * kq + (gq >> 1);
      const int at = PS_Q + tok * 256 + 8 * (gq & 1);
      cq[n][0] = lds_at<uint2>(lb, at + ((cc ^ m) << 4));
      cq[n][1] = lds_at<uint2>(lb, at + (((cc + 2) ^ m) << 4));
    }
  }
  f32x4 acc[4];
  int jrb[NJ], jcb[NJ];
  bool jqk[NJ];
  if (wave == 0) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      acc[b] = zero4();
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const bf16x8 f = pfrag16(lb, PS_K, 16 * b, kk, L);
        acc[b] = mfma(f, f, acc[b]);
      }
    }
  } else {
#pragma unroll
    for (int n = 0; n < NJ; ++n) {
      const int j = wave - 1 + (W - 1) * n;
      jrb[n] = jcb[n] = 0;
      jqk[n] = false;
      acc[n] = zero4();
      if (j < 16) {
        int rb, cb;
        if (j < 6) {
          rb = j < 1 ? 1 : (j < 3 ? 2 : 3);
          cb = j - rb * (rb - 1) / 2;
        } else {
          lower_tile(j - 6, rb, cb);
        }
        jrb[n] = rb;
        jcb[n] = cb;
        jqk[n] = j >= 6;
        const int am = j >= 6 ? PS_Q : PS_K;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
          acc[n] = mfma(pfrag16(lb, am, 16 * rb, kk, L), pfrag16(lb, PS_K, 16 * cb, kk, L), acc[n]);
      }
    }
  }
  item_barrier();  // A^T overwrites the q rows; the factors are visible

  // 3. scaled tiles -> A^T (fp32) and P^T (bf16); wave 0: the diagonal blocks, then their inverse
  // A_ij = beta_i rk_i exp(G_i - G_j) rk_j k_i.k_j (i > j), P_ij = s rq_i exp(G_i - G_j) rk_j q_i.k_j (i >= j),
  // each factor as one exp2(u_i - h_j): u_i = log2(beta_i rk_i) + G_i log2(e) (A) or log2(s rq_i) +
  // G_i log2(e) (P), h_j = G_j log2(e) - log2(rk_j); only the diagonal tiles need the triangle mask
  auto scale_tile = [&](f32x4 a, int rb, int cb, bool qk) {
    const int j = 16 * cb + m, i0 = 16 * rb + 4 * gq;
    const float hj = F[(PSF_H >> 2) + j];
    const f32x4 u4 = lds_at<f32x4>(lb, PS_F + (qk ? PSF_UP : PSF_UA) + 4 * i0);
    f32x4 e;
#pragma unroll
    for (int r = 0; r < 4; ++r) e[r] = a[r] * __builtin_amdgcn_exp2f(u4[r] - hj);
    if (rb == cb) {  // (wave-uniform)
#pragma unroll
      for (int r = 0; r < 4; ++r) e[r] = (qk ? i0 + r >= j : i0 + r > j) ? e[r] : 0.f;
    }
    return e;
  };
  if (wave == 0) {
#pragma unroll
    for (int b = 0; b < 4; ++b) put_t32(lb, PS_AT, b, b, L, scale_tile(acc[b], b, b, false));
    wave_sync_lds();
    // right-looking substitution: lane (block gq, column m); s[r] -> T_b[r][m]
    float sv[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) sv[r] = r == m ? 1.f : 0.f;
    const int rowb = PS_AT + gq * 4096 + ((4 * gq) << 4);  // row 16 gq of A^T, chunk 4 gq (before the XORs)
    // the row of A^T for step mm (column mm of the block) is read one step ahead, only its chunks that hold
    // rows below mm
    f32x4 a4[4], n4[4];
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) a4[qd] = lds_at<f32x4>(lb, (rowb ^ (qd << 4)));
#pragma unroll
    for (int mm = 0; mm < 15; ++mm) {
#pragma unroll
      for (int qd = 0; qd < 4; ++qd)
        if (mm + 1 < 15 && 4 * qd + 3 > mm + 1) n4[qd] = lds_at<f32x4>(lb, (rowb ^ ((qd ^ (mm + 1)) << 4)) + (mm + 1) * 256);
      const float t = sv[mm];
#pragma unroll
      for (int r = mm + 1; r < 16; ++r) sv[r] = fmaf(-a4[r >> 2][r & 3], t, sv[r]);
#pragma unroll
      for (int qd = 0; qd < 4; ++qd)
        if (4 * qd + 3 > mm + 1) a4[qd] = n4[qd];
    }
    // column m of T_b -> row 16 gq + m of T^T, columns 16 gq .. + 15
    const int roww = PS_TT + (16 * gq + m) * 256 + (((4 * gq) ^ m) << 4);
#pragma unroll
    for (int qd = 0; qd < 4; ++qd)
      lds_put<f32x4>(lb, roww ^ (qd << 4), f32x4{sv[4 * qd], sv[4 * qd + 1], sv[4 * qd + 2], sv[4 * qd + 3]});
  } else {
#pragma unroll
    for (int n = 0; n < NJ; ++n) {
      if (wave - 1 + (W - 1) * n < 16) {
        const f32x4 e = scale_tile(acc[n], jrb[n], jcb[n], jqk[n]);
        if (jqk[n]) put_t16(lb, PS_PT, jrb[n], jcb[n], L, e);
        else put_t32(lb, PS_AT, jrb[n], jcb[n], L, e);
      }
    }
  }
  item_barrier();

  // 4. off-diagonal blocks of T: N_ij = T_ii A_ij (i > j, into A's blocks), then T_10, T_21, T_32 and the
  // pair products N_21 N_10, N_32 N_20, N_32 N_21 (into T's blocks (0, 1..3)), then T_20, T_31, T_30
  if (wave < 6) {
    const int i = wave < 1 ? 1 : (wave < 3 ? 2 : 3), j = wave - i * (i - 1) / 2;
    put_t32(lb, PS_AT, i, j, L, mm_t(lb, PS_TT, i, i, PS_AT, i, j, L, zero4()));
  }
  item_barrier();
  if (wave < 3) {
    put_t32(lb, PS_TT, wave + 1, wave, L, -mm_t(lb, PS_AT, wave + 1, wave, PS_TT, wave, wave, L, zero4()));
  } else if (wave < 6) {
    const int ai = wave == 3 ? 2 : 3, aj = wave == 3 ? 1 : 2, ci = wave == 3 ? 1 : 2, cj = wave == 5 ? 1 : 0;
    put_t32(lb, PS_TT, 0, wave - 2, L, mm_t(lb, PS_AT, ai, aj, PS_AT, ci, cj, L, zero4()));
  }
  item_barrier();
  if (wave == 0) {
    put_t32(lb, PS_TT, 2, 0, L, mm_t_diff(lb, PS_TT, 0, 1, PS_AT, 2, 0, PS_TT, 0, 0, L, zero4()));
  } else if (wave == 1) {
    put_t32(lb, PS_TT, 3, 1, L, mm_t_diff(lb, PS_TT, 0, 3, PS_AT, 3, 1, PS_TT, 1, 1, L, zero4()));
  } else if (wave == 2) {
    f32x4 t = mm_t_diff(lb, PS_TT, 0, 2, PS_AT, 3, 0, PS_TT, 0, 0, L, zero4());
    t = mm_t_diff(lb, PS_TT, 0, 3, PS_AT, 3, 1, PS_TT, 1, 0, L, t);
    put_t32(lb, PS_TT, 3, 0, L, t);
  }
  item_barrier();

  // 5. bf16 forms, row by row of T^T (row j = column j of T; 8 columns i0 .. i0 + 7 a thread):
  // TBF^T[j][i] = Fk_i T_ij... = Fk_i T[i][j] Bk_j, TBT[j][i] = T[i][j] Bk_j, LB^T[j][i] = (T - I)[i][j] beta_j;
  // T's blocks above its diagonal blocks (pair products there) are zero
  {
    const bool act = W == 8 || tid < 512;  // (512 threads: 8 a row of T^T)
    const int j = (tid >> 3) & 63, i0 = (tid & 7) * 8;
    const int rd = PS_TT + j * 256 + (((2 * (tid & 7)) ^ (j & 15)) << 4);
    f32x4 t0 = lds_at<f32x4>(lb, rd), t1 = lds_at<f32x4>(lb, rd ^ 16);
    if ((i0 >> 4) < (j >> 4)) t0 = t1 = zero4();
    const float bkj = F[(PSF_BK >> 2) + j], bj = F[(PSF_B >> 2) + j];
    const f32x4 fk0 = lds_at<f32x4>(lb, PS_F + PSF_FK + 4 * i0), fk1 = lds_at<f32x4>(lb, PS_F + PSF_FK + 4 * i0 + 16);
    const float tv[8] = {t0[0], t0[1], t0[2], t0[3], t1[0], t1[1], t1[2], t1[3]};
    const float fk[8] = {fk0[0], fk0[1], fk0[2], fk0[3], fk1[0], fk1[1], fk1[2], fk1[3]};
    uint32_t wf[4], wt[4], wl[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const float b0 = tv[2 * p] * bkj, b1 = tv[2 * p + 1] * bkj;
      wf[p] = pack_bf16x2(fk[2 * p] * b0, fk[2 * p + 1] * b1);
      wt[p] = pack_bf16x2(b0, b1);
      wl[p] = pack_bf16x2(i0 + 2 * p == j ? 0.f : tv[2 * p] * bj, i0 + 2 * p + 1 == j ? 0.f : tv[2 * p + 1] * bj);
    }
    item_barrier();  // the forms overwrite T^T and A^T
    const int wr = j * 128 + ((((tid & 7) ^ ((j >> 1) & 7))) << 4);
    if (act) {
      lds_put<uint4>(lb, PS_TBF + wr, make_uint4(wf[0], wf[1], wf[2], wf[3]));
      lds_put<uint4>(lb, PS_TBT + wr, make_uint4(wt[0], wt[1], wt[2], wt[3]));
      lds_put<uint4>(lb, PS_LB + wr, make_uint4(wl[0], wl[1], wl[2], wl[3]));
    }
  }
  item_barrier();

  if constexpr (!QL) {
#pragma unroll
    for (int n = 0; n < NJ16; ++n) {
      const int job = wave + W * n, tb = job >> 2, kq = job & 3;
      const int tok = 16 * tb + m;
      cq[n][0] = cq[n][1] = make_uint2(0, 0);
      if (tok < cr.len) {
        const uint16_t* qrow = q + (size_t)(cr.t0 + tok) * rs.q + hk * DK + 32 * kq + 4 * gq;
        cq[n][0] = *reinterpret_cast<const uint2*>(qrow);
        cq[n][1] = *reinterpret_cast<const uint2*>(qrow + 16);
      }
    }
  }

  // 6. W'^T = K^T TBF^T (A fragments to the workspace), R = P TB (as R^T; R's blocks above its diagonal
  // blocks zero), the K^T fragments
  {
    uint4* gW = reinterpret_cast<uint4*>(wsc + WS_WP);
#pragma unroll
    for (int n = 0; n < NJ16; ++n) {
      const int job = wave + W * n, tb = job >> 2, kq = job & 3, nk = tri_kend(tb) / 32;
      f32x4 d0 = zero4(), d1 = zero4();
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
        if (kk < nk) {
          const bf16x8 bf = pfragT8(lb, PS_TBF, 16 * tb, kk, L);
          d0 = mfma(pfragT16(lb, PS_K, 32 * kq, kk, L), bf, d0);
          d1 = mfma(pfragT16(lb, PS_K, 32 * kq + 16, kk, L), bf, d1);
        }
      gW[(tb * 4 + kq) * 64 + l] = kappa_frag(d0, d1);
    }
#pragma unroll
    for (int n = 0; n < NJ16; ++n) {  // R tiles: jobs 0-9 the lower tiles, 10-15 zero tiles above
      const int job = wave + W * n;
      int rb, cb;
      if (job < 10) {
        lower_tile(job, rb, cb);
        f32x4 r = zero4();
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
          if (kk < tri_kend(rb) / 32) r = mfma(pfragT8(lb, PS_PT, 16 * rb, kk, L), pfrag8(lb, PS_TBT, 16 * cb, kk, L), r);
        put_t16(lb, PS_RT, rb, cb, L, r);
      } else {
        const int t = job - 10;  // (rb, cb) with rb < cb: (0,1) (0,2) (1,2) (0,3) (1,3) (2,3)
        cb = t < 1 ? 1 : (t < 3 ? 2 : 3);
        rb = t - cb * (cb - 1) / 2;
        put_t16(lb, PS_RT, rb, cb, L, zero4());
      }
    }
    uint4* gKT = reinterpret_cast<uint4*>(wsc + WS_KT);
#pragma unroll
    for (int n = 0; n < NJ16; ++n) {  // fragment f = 2 w + kk = wave + W n (16 fragments of 64 lanes)
      const int f = wave + W * n;
      gKT[f * 64 + l] = __builtin_bit_cast(uint4, pfragT16(lb, PS_K, 16 * (f >> 1), f & 1, L));
    }
  }
  item_barrier();  // Ub^T overwrites TBF, TBT

  // 7. Ub = beta V + LB V: Ub' = Fk Ub (fp32 D tiles) to the workspace, Ub^T (bf16) to LDS
  {
    float4* gU = reinterpret_cast<float4*>(wsc + WS_UB);
    const int vb = wave & 7;
#pragma unroll
    for (int tt = 0; tt < TBN; ++tt) {
      const int tb = (wave >> 3) * TBN + tt;
      f32x4 u = zero4();
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
        if (kk < tri_kend(tb) / 32) u = mfma(pfragT8(lb, PS_LB, 16 * tb, kk, L), pfragT16(lb, PS_V, 16 * vb, kk, L), u);
      const int i0 = 16 * tb + 4 * gq;
      const uint2 vv = lds_tr(lb, PS_V + 4096 * tb + (L.dv ^ (32 * vb)));
      const f32x4 bs = lds_at<f32x4>(lb, PS_F + PSF_B + 4 * i0);
      const f32x4 fk = lds_at<f32x4>(lb, PS_F + PSF_FK + 4 * i0);
      f32x4 ub;
      ub[0] = fmaf(bs[0], __uint_as_float(vv.x << 16), u[0]);
      ub[1] = fmaf(bs[1], __uint_as_float(vv.x & 0xffff0000u), u[1]);
      ub[2] = fmaf(bs[2], __uint_as_float(vv.y << 16), u[2]);
      ub[3] = fmaf(bs[3], __uint_as_float(vv.y & 0xffff0000u), u[3]);
      gU[(vb * 4 + tb) * 64 + l] = make_float4(fk[0] * ub[0], fk[1] * ub[1], fk[2] * ub[2], fk[3] * ub[3]);
      put_t16(lb, PS_UBT, tb, vb, L, ub);
    }
  }
  item_barrier();

  // 8. Q' = Fq q - R K (as A fragments) and Ob = P Ub (bf16 D tiles); G_L
  {
    uint4* gQ = reinterpret_cast<uint4*>(wsc + WS_QP);
#pragma unroll
    for (int n = 0; n < NJ16; ++n) {
      const int job = wave + W * n, tb = job >> 2, kq = job & 3, nk = tri_kend(tb) / 32;
      f32x4 d0 = zero4(), d1 = zero4();
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
        if (kk < nk) {
          const bf16x8 rf = pfragT8(lb, PS_RT, 16 * tb, kk, L);
          d0 = mfma(pfragT16(lb, PS_K, 32 * kq, kk, L), rf, d0);
          d1 = mfma(pfragT16(lb, PS_K, 32 * kq + 16, kk, L), rf, d1);
        }
      const float fq = F[(PSF_FQ >> 2) + 16 * tb + m];
      const uint2 c0 = cq[n][0], c1 = cq[n][1];
      d0[0] = fmaf(fq, __uint_as_float(c0.x << 16), -d0[0]);
      d0[1] = fmaf(fq, __uint_as_float(c0.x & 0xffff0000u), -d0[1]);
      d0[2] = fmaf(fq, __uint_as_float(c0.y << 16), -d0[2]);
      d0[3] = fmaf(fq, __uint_as_float(c0.y & 0xffff0000u), -d0[3]);
      d1[0] = fmaf(fq, __uint_as_float(c1.x << 16), -d1[0]);
      d1[1] = fmaf(fq, __uint_as_float(c1.x & 0xffff0000u), -d1[1]);
      d1[2] = fmaf(fq, __uint_as_float(c1.y << 16), -d1[2]);
      d1[3] = fmaf(fq, __uint_as_float(c1.y & 0xffff0000u), -d1[3]);
      gQ[(tb * 4 + kq) * 64 + l] = kappa_frag(d0, d1);
    }
    uint2* gO = reinterpret_cast<uint2*>(wsc + WS_OB);
    const int vb = wave & 7;
#pragma unroll
    for (int tt = 0; tt < TBN; ++tt) {
      const int tb = (wave >> 3) * TBN + tt;
      f32x4 y = zero4();
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
        if (kk < tri_kend(tb) / 32) y = mfma(pfragT8(lb, PS_PT, 16 * tb, kk, L), pfrag8(lb, PS_UBT, 16 * vb, kk, L), y);
      gO[(vb * 4 + tb) * 64 + l] = make_uint2(pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3]));
    }
    if (tid == 0) *reinterpret_cast<float*>(wsc + WS_GL) = F[(PSF_G >> 2) + CH - 1];
  }
  item_barrier();  // the next item's rows overwrite the LDS
}

// Per-thread constants of the item's row loads: LDS offset of row rr (and rr + 32) at columns c8 .. and
// the rows' byte offsets in the q, k, v buffers.
struct PrepRows {
  int rowoff;
  uint32_t oq, ok, ov;
  __device__ __forceinline__ PrepRows(int tid, const RowStrides& rs) {
    const int rr = tid >> 4, cc = tid & 15;
    rowoff = rr * 256 + ((cc ^ (rr & 15)) << 4);
    oq = (uint32_t)rr * 2u * (uint32_t)rs.q + 16u * cc;
    ok = (uint32_t)rr * 2u * (uint32_t)rs.k + 16u * cc;
    ov = (uint32_t)rr * 2u * (uint32_t)rs.v + 16u * cc;
  }
};

// W = 8: two workgroups a CU; W = 16: one (the same registers a wave).
template <typename TG, bool GATE, int W>
__global__ __launch_bounds__(64 * W, P1_WAVES_PER_SIMD) void chunk_prep_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const TG* __restrict__ g, const TG* __restrict__ beta, const float* __restrict__ A_log,
    const float* __restrict__ dt_bias, const int32_t* __restrict__ cu, const int32_t* __restrict__ chunk_idx,
    int n_seqs, int n_items, int T, int Hk, int Hv, float scale, int qk_l2norm, const RowStrides rs,
    uint8_t* __restrict__ ws) {
  __shared__ PrepShared sm;
  uint8_t* lb = sm.b;
  const PrepLane L(lane_id());
  const PrepRows lr(threadIdx.x, rs);
  prep_init(lb);
  RowRegs R;
  ItemWalk w(blockIdx.x, gridDim.x, Hv, Hk, T);
  if (w.item >= n_items) return;
  ItemAt cur = w.at(cu, chunk_idx, n_seqs, T);  // (a packed batch's chunk table is read for items < n_items only)
  load_rows<W>(R, cur, q, k, v, rs, lr.oq, lr.ok, lr.ov);
  while (w.item < n_items) {
    w.advance();
    const bool has_next = w.item < n_items;
    ItemAt nx = cur;
    if (has_next) nx = w.at(cu, chunk_idx, n_seqs, T);
    prep_item<TG, GATE, true, W>(lb, cur, R, has_next, nx, q, k, v, g, beta, A_log, dt_bias, Hv, scale, qk_l2norm, rs, ws, L,
                        lr.rowoff, lr.oq, lr.ok, lr.ov);
    cur = nx;
  }
}

// ----------------------------------------------------------------------------------------------- phase 2

constexpr int P2_WAVES = 8;

// LDS-only workgroup barrier: waits for this wave's LDS traffic, not for its outstanding global loads
// (the prefetch of the next chunk stays in flight across it).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Operands of one chunk held in registers (prefetched one chunk ahead), for a workgroup of NV value blocks.
template <int NV>
struct Pre {
  bf16x8 A[4];   // W' (U role) or Q' (O role) fragments of this wave's 16 tokens, k-steps 0..3
  bf16x8 KT[2];  // K^T fragments of this wave's 16 state columns, token steps 0, 1
  uint4 X[NV];   // per value block, U role: Ub' (4 fp32); O role: Ob (4 bf16 in .x, .y)
  float GL;      // G at the chunk end
};

// Single buffers suffice: each is rewritten only after a barrier that every reader of it has passed.
// The state slice sits in 256-byte rows with 16-byte chunk c of row r at chunk c ^ r (r < 16): its fragment
// reads (16 rows at one chunk) then meet every bank once. (With padded 272-byte rows each of those reads took
// 8 LDS cycles, 4 of them bank conflicts, against 4 and none: measured with the hardware counters.)
template <int NV>
struct StateSharedT {
  uint16_t Ss[NV * VB * DK];   // state slice (bf16), key columns at positions pi(key): B operand of [W'; Q'] S^T
  uint16_t UhT[NV * VB][LDC];  // U'^T, hi part   } A operands of the state update
  uint16_t UlT[NV * VB][LDC];  // U'^T, lo part   }
};
using StateShared = StateSharedT<1>;
__device__ __forceinline__ int ss_at(int r, int c) { return r * DK + ((((c >> 3) ^ r) & 15) << 3) + (c & 7); }

struct StateArgs {
  const uint8_t* ws;
  int c0, bos, len, nchunks, Hv, h, vb;
  float xs;  // 1, or 0 for a transition run (Ub' and Ob taken as zero: the pass then carries S -> S A_c)
  // overlapped form: the ready flag of this job's chunk ci is flags[ci * flag_step], nonzero once phase 1 has
  // stored the item (flag_step 0 with flags on a word that stays zero: every wait runs out -- the host's test
  // of the error path); spin_max bounds each wait
  const int* flags;
  int flag_step;
  int spin_max;
};

// Default bound on a state pass's wait for one item (a few tenths of a second): a wait that runs out sets bit
// ZGDN_STATUS_WAIT_GAVE_UP of the device status word, and the wave then waits no more, so that every wave of
// the kernel ends soon.
constexpr int SPIN_MAX = 1 << 17;

// Sticky device status of this library's chunked-prefill kernels on each device (bits of zgdn_chunk_status),
// read and cleared by zgdn_chunk_status.
__device__ int g_chunk_status;

__device__ __forceinline__ int load_flag(const int* f) {
  return __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}


// Stores one O wave's outputs of chunk ci: rows t0 .. t0+3 (D layout) of value column vb * VB + j. Lanes l and
// l ^ 1 (adjacent columns) swap two values by DPP so that each stores two rows as column pairs, 4-byte words
// (8 for fp32) instead of 2-byte ones. The stores go through a buffer resource covering the chunk's rows of
// this job's columns up to the chunk's last token, so rows past the end of a partial chunk are dropped by the
// range check instead of a per-row condition.
template <typename TOut>
__device__ __forceinline__ void store_o_tile(TOut* o, const StateArgs& a, int vb, int ci, int t0, int j,
                                             const float* ov) {
  const bool odd = (lane_id() & 1) != 0;
  const float r0 = dpp<DPP_QUAD_XOR1>(odd ? ov[0] : ov[2]), r1 = dpp<DPP_QUAD_XOR1>(odd ? ov[1] : ov[3]);
  // even lane (column j): rows t0, t0+1 as (own, partner); odd lane (column j): rows t0+2, t0+3 as (partner, own)
  const float a0 = odd ? r0 : ov[0], b0 = odd ? ov[2] : r0, a1 = odd ? r1 : ov[1], b1 = odd ? ov[3] : r1;
  const int tr = t0 + (odd ? 2 : 0), tlen = min(CH, a.len - ci * CH);
  const uint32_t row = (uint32_t)a.Hv * DV * (uint32_t)sizeof(TOut);  // bytes from one token to the next
  const Rsrc r = raw_rsrc(o + ((size_t)(a.bos + ci * CH) * a.Hv + a.h) * DV + vb * VB, (uint32_t)tlen * row);
  const uint32_t off = (uint32_t)tr * row + (uint32_t)(j & ~1) * (uint32_t)sizeof(TOut);
  if constexpr (sizeof(TOut) == 2) {
    __builtin_amdgcn_raw_buffer_store_b32(pack_bf16x2(a0, b0), r, off, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b32(pack_bf16x2(a1, b1), r, off + row, 0, 0);
  } else {
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(a0), __float_as_uint(b0)}, r, off, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(a1), __float_as_uint(b1)}, r, off + row, 0, 0);
  }
}

// The chunk loop of one wave. URole: waves 0-3 form U' = Ub' - W' S^T of their 16 tokens; the O role
// (waves 4-7) forms the outputs O = Ob + Q' S^T of their 16 tokens. Both run the same barriers and each
// wave updates 16 columns of the state slice. The slice holds NV blocks of 16 value rows (a.vb .. a.vb + NV -
// 1): every operand fetched for a chunk but Ub' / Ob serves all of them.
template <bool URole, typename TOut, bool Wait, int NV>
__device__ __forceinline__ void state_loop(StateSharedT<NV>& sh, const StateArgs& a, TOut* o, f32x4 (&S)[NV]) {
  const int l = lane_id(), wave = threadIdx.x >> 6;
  const int tb = wave & 3;               // this wave's token tile
  const int j = l & 15;                  // value row within the slice (D layout column of [W'; Q'] S^T)
  const int t0 = 16 * tb + 4 * (l >> 4);  // first of this lane's 4 tokens (D layout rows)
  // position of key column 16 wave + l%16 in Ss, the inverse of kappa
  const int pcol = 32 * (wave >> 1) + 8 * ((l & 15) >> 2) + 4 * (wave & 1) + (l & 3);
  // this lane's Ss addresses, the same for every chunk: its 4 state elements (rows 4 (l/16) + i4, column
  // pcol) and its fragments (row l%16, columns 32 kk + 8 (l/16) ..)
  // (the fragment addresses in 16-byte chunks, so that the compiler sees their alignment and keeps each read
  // one 16-byte access)
  // (block v of the slice at rows 16 v ..: + 16 v DK elements, 2 v DK 16-byte chunks)
  int ss_w[4], ss_r[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    ss_w[i] = ss_at(4 * (l >> 4) + i, pcol);
    ss_r[i] = ss_at(l & 15, 32 * i + 8 * (l >> 4)) >> 3;
  }
  const bf16x8* ss_chunks = reinterpret_cast<const bf16x8*>(sh.Ss);

  // a chunk's workspace as a buffer resource (scalar registers, formed per chunk)
  auto chunk_ws = [&](int ci) { return raw_rsrc(a.ws + ((size_t)(a.c0 + ci) * a.Hv + a.h) * WS_CHUNK, WS_CHUNK); };
  // per-lane byte offsets inside a chunk's workspace, the same for every chunk
  const uint32_t offA = (uint32_t)(URole ? WS_WP : WS_QP) + (uint32_t)(tb * 4 * 64 + l) * 16u;
  const uint32_t offX = URole ? (uint32_t)WS_UB + (uint32_t)((a.vb * 4 + tb) * 64 + l) * 16u
                              : (uint32_t)WS_OB + (uint32_t)((a.vb * 4 + tb) * 64 + l) * 8u;
  constexpr uint32_t XB = URole ? 4u * 64u * 16u : 4u * 64u * 8u;  // from one value block's Ub' / Ob to the next
  const uint32_t offK = (uint32_t)WS_KT + (uint32_t)(wave * 2 * 64 + l) * 16u;
  auto ld16 = [](Rsrc w, uint32_t off) {
    return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(w, off, 0, 0));
  };
  // the next chunk's loads in groups spread over the phases of the current chunk
  auto fetch1 = [&](Rsrc w, Pre<NV>& x) {
    x.A[0] = ld16(w, offA);
    x.A[1] = ld16(w, offA + 1024u);
    x.GL = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(w, 0, (int)WS_GL, 0));
  };
  auto fetch2 = [&](Rsrc w, Pre<NV>& x) {
    x.A[2] = ld16(w, offA + 2048u);
    x.A[3] = ld16(w, offA + 3072u);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      if constexpr (URole) {
        x.X[v] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(w, offX + v * XB, 0, 0));
      } else {
        const uint2 ob = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(w, offX + v * XB, 0, 0));
        x.X[v] = make_uint4(ob.x, ob.y, 0, 0);
      }
    }
  };
  auto fetch3 = [&](Rsrc w, Pre<NV>& x) {
    x.KT[0] = ld16(w, offK);
    x.KT[1] = ld16(w, offK + 1024u);
  };

  // Overlapped form: before the loads of chunk ni, wait for its ready flag (read one chunk ahead, so that
  // the flag's round trip is hidden when phase 1 is ahead) and issue the read of the next one's.
  if (a.nchunks <= 0) return;
  const int last = a.nchunks - 1;
  const int* fbase = Wait ? a.flags : nullptr;
  int fl = 0;
  bool gave_up = false;
  auto wait_ready = [&](int ni) {
    if constexpr (Wait) {
      int f = gave_up ? 1 : fl;
      for (int n = 0; f == 0; ++n) {
        if (n >= a.spin_max) {
          if (l == 0)
            __hip_atomic_fetch_or(&g_chunk_status, ZGDN_STATUS_WAIT_GAVE_UP, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
          gave_up = true;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
        f = load_flag(fbase + (size_t)ni * a.flag_step);
      }
      asm volatile("" ::: "memory");  // the chunk's loads stay behind the wait
      fl = load_flag(fbase + (size_t)min(ni + 1, last) * a.flag_step);
    }
  };

  auto process = [&](int ci, const Pre<NV>& cur, int ni, Pre<NV>& nxt) {
#pragma unroll
    for (int v = 0; v < NV; ++v)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) sh.Ss[v * VB * DK + ss_w[i4]] = f32_to_bf16(S[v][i4]);
    wait_ready(ni);
    const Rsrc wn = chunk_ws(ni);
    fetch1(wn, nxt);
    lds_barrier();

    float ov[NV][4];  // O role: this wave's outputs
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      // [W'; Q'] S^T for this wave's 16 tokens, as two independent MFMA chains (half the dependent latency)
      f32x4 x0 = zero4(), x1 = zero4();
#pragma unroll
      for (int kk = 0; kk < 4; kk += 2) {
        x0 = mfma(cur.A[kk], ss_chunks[v * VB * DK / 8 + ss_r[kk]], x0);
        x1 = mfma(cur.A[kk + 1], ss_chunks[v * VB * DK / 8 + ss_r[kk + 1]], x1);
      }
      const f32x4 x = x0 + x1;
      const uint4 X = cur.X[v];
      if constexpr (URole) {
        // U' = Ub' - W' S^T as hi + lo bf16
        const float ub[4] = {a.xs * __uint_as_float(X.x), a.xs * __uint_as_float(X.y), a.xs * __uint_as_float(X.z),
                             a.xs * __uint_as_float(X.w)};
        float u[4];
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) u[i4] = ub[i4] - x[i4];
        const uint32_t h01 = pack_bf16x2(u[0], u[1]), h23 = pack_bf16x2(u[2], u[3]);
        const uint32_t l01 = pack_bf16x2(u[0] - __uint_as_float(h01 << 16), u[1] - __uint_as_float(h01 & 0xffff0000u));
        const uint32_t l23 = pack_bf16x2(u[2] - __uint_as_float(h23 << 16), u[3] - __uint_as_float(h23 & 0xffff0000u));
        *reinterpret_cast<uint2*>(&sh.UhT[v * VB + j][t0]) = make_uint2(h01, h23);
        *reinterpret_cast<uint2*>(&sh.UlT[v * VB + j][t0]) = make_uint2(l01, l23);
      } else {
        // O = Ob + Q' S^T (stored after the state update is issued)
        const float ob[4] = {a.xs * __uint_as_float(X.x << 16), a.xs * __uint_as_float(X.x & 0xffff0000u),
                             a.xs * __uint_as_float(X.y << 16), a.xs * __uint_as_float(X.y & 0xffff0000u)};
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) ov[v][i4] = ob[i4] + x[i4];
      }
    }
    fetch2(wn, nxt);
    lds_barrier();
    // (the next chunk's K^T fragments are not needed before the next update: issued past the barrier, so that
    // their issue is off the barrier's path; 71.8-71.9 against 73.7-73.9 us at T = 4096, 16 heads)
    fetch3(wn, nxt);

    // S <- exp(G_L) S + U'^T K for this wave's 16 columns (two chains over the key steps)
    const float decay = __expf(cur.GL);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      f32x4 acc0 = S[v] * decay, acc1 = zero4();
      acc0 = mfma(frag(&sh.UhT[v * VB][0], LDC, 0, 0), cur.KT[0], acc0);
      acc1 = mfma(frag(&sh.UhT[v * VB][0], LDC, 0, 32), cur.KT[1], acc1);
      acc0 = mfma(frag(&sh.UlT[v * VB][0], LDC, 0, 0), cur.KT[0], acc0);
      acc1 = mfma(frag(&sh.UlT[v * VB][0], LDC, 0, 32), cur.KT[1], acc1);
      S[v] = acc0 + acc1;
    }
    if constexpr (!URole) {
#pragma unroll
      for (int v = 0; v < NV; ++v) store_o_tile(o, a, a.vb + v, ci, t0, j, ov[v]);
    }
  };

  // two register buffers, alternately filled one chunk ahead (no copies between them). The fetches are
  // unconditional (the last chunk is fetched again at the end) so every path issues the same loads, and the
  // first chunk is peeled so that the loop is entered with the same loads in flight as at its back edge
  // (which keeps the compiler's wait counts at the loop head from covering the prefetch). (Fetching two
  // chunks ahead, with a third buffer, measured no faster: the loop is bound by the per-CU load rate, not by
  // memory latency.)
  Pre<NV> b0, b1;
  {
    if constexpr (Wait) fl = load_flag(fbase);
    wait_ready(0);
    const Rsrc w0 = chunk_ws(0);
    fetch1(w0, b0);
    fetch2(w0, b0);
    fetch3(w0, b0);
  }
  process(0, b0, min(1, last), b1);
  int ci = 1;
  for (; ci + 1 < a.nchunks; ci += 2) {
    process(ci, b1, ci + 1, b0);
    process(ci + 1, b0, min(ci + 2, last), b1);
  }
  if (ci < a.nchunks) process(ci, b1, ci, b0);
}

// Segmented runs of phase 2 (unpacked batches whose pass would hold few CUs): each sequence is cut into G
// segments of Cs chunks. "Local" runs carry each segment from a zero state (the first from the sequence's
// initial state) and write its outputs and end state L_g; "transition" runs carry segments 1.. from the
// identity with Ub' = Ob = 0, so their state is the segment's map P_c = A_1 .. A_c (S -> S A_c per chunk), their
// end state M_g and their outputs Q'_c P_c^T. The true state entering segment g is S_g = S_{g-1} M_{g-1} +
// L_{g-1} (S_1 = L_0) and the true outputs are o_local + (Q' P^T) S_g^T: chunk_combine_kernel and
// chunk_correct_kernel form them. All local and transition workgroups run at once.
struct SegRun {
  int G, Cs;               // segments per sequence, chunks per segment (G == 1: plain runs)
  float* local_final;      // L [n_seqs * G][Hv][V][K]
  float* trans_final;      // M^T [n_seqs * (G - 1)][Hv] as bf16 hi then lo, each [K][K] in mt_frag order
  uint16_t* trans_out;     // Q' P^T [n_seqs * T][Hv][K] (bf16)
};

// Position (in 16-bit elements) of M^T[n][k] in the transition runs' stored maps: the order in which
// chunk_combine_kernel's waves read them as MFMA B fragments -- fragment (w, t, kb) (columns n = 32 w + 16 t ..
// + 15 of M, keys k = 32 kb ..) as 64 lanes x 8 elements, lane 16 ((k >> 3) & 3) + n % 16 holding keys
// k & ~7 .. + 7 -- so that each fragment load is 1 KiB of contiguous memory. (Read as rows of M^T, a fragment
// touched 16 rows per instruction, a third of the rate of contiguous reads.) Four consecutive keys k .. k + 3
// (k % 4 == 0) are contiguous.
__device__ __forceinline__ size_t mt_frag(int n, int k) {
  const int w = n >> 5, t = (n >> 4) & 1, kb = k >> 5, g = (k >> 3) & 3;
  return ((size_t)((w * 2 + t) * (DK / 32) + kb) * 64 + 16 * g + (n & 15)) * 8 + (k & 7);
}

template <typename TOut, int NV>
__global__ __launch_bounds__(64 * P2_WAVES) void chunk_state_kernel(
    const uint8_t* ws, const float* __restrict__ s_in, float* __restrict__ s_out, TOut* __restrict__ o,
    const int32_t* __restrict__ cu, int n_seqs, int n_chunks, int T, int Hv, const SegRun seg) {
  // (ws is not __restrict__: that keeps the compiler from sinking the prefetch loads below the LDS
  // barriers, whose asm memory clobber then pins them where they are issued)
  __shared__ StateSharedT<NV> sh;
  constexpr int NG = DV / VB / NV;  // workgroups per (run, head): NV value blocks of 16 rows each

  // XCD-aware order (workgroups go round-robin over the 8 XCDs): ids are taken in groups of 8 NG = 8 pairs
  // (run, head) x NG value-block groups, with id % 8 = pair % 8, so the NG workgroups of one pair run on one
  // XCD at the same time and share its L2 copy of the chunk workspace. The grid is padded to whole groups.
  const int n_local = n_seqs * seg.G * Hv, n_trans = n_seqs * (seg.G - 1) * Hv;
  const int id = blockIdx.x;
  const int pair = (id / (8 * NG)) * 8 + (id % 8), vb = ((id % (8 * NG)) / 8) * NV;  // first value block
  if (pair >= n_local + n_trans) return;
  const bool trans = pair >= n_local;
  const int vp = trans ? pair - n_local : pair;
  const int h = vp % Hv, run = vp / Hv;  // run: the (sequence, segment) index among local / transition runs
  const int seq = trans ? run / (seg.G - 1) : run / seg.G;
  const int sg = trans ? 1 + run % (seg.G - 1) : run % seg.G;
  const int l = lane_id(), wave = threadIdx.x >> 6;
  const int ncol = 16 * wave + (l & 15);

  StateArgs a;
  a.ws = ws;
  a.Hv = Hv;
  a.h = h;
  a.vb = vb;
  a.xs = trans ? 0.f : 1.f;
  if (cu != nullptr) {  // packed sequences: plain runs only
    int eos;
    seq_bounds(cu, seq, T, a.bos, eos);
    a.len = eos - a.bos;
    a.c0 = 0;
    for (int s = 0; s < seq; ++s) {
      int sb, se;
      seq_bounds(cu, s, T, sb, se);
      a.c0 += (se - sb + CH - 1) / CH;
    }
  } else {
    const int nct = (T + CH - 1) / CH;
    a.bos = seq * T + sg * seg.Cs * CH;
    a.len = min(seg.Cs * CH, T - sg * seg.Cs * CH);
    a.c0 = seq * nct + sg * seg.Cs;
  }
  // chunks past the workspace (a chunk table shorter than the sequences need) are not read
  a.nchunks = max(0, min((a.len + CH - 1) / CH, n_chunks - a.c0));

  // state slice in the D layout of the state update: block v, rows j = 4*(l/16)+i, column ncol
  f32x4 S[NV];
  const size_t hs = (size_t)DV * DK;
  auto slice = [&](int v) { return ((size_t)(vb + v) * VB + 4 * (l >> 4)) * DK + ncol; };  // within a [V][K] state
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    if (trans) {
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) S[v][i4] = (vb + v) * VB + 4 * (l >> 4) + i4 == ncol ? 1.f : 0.f;
    } else {
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4)
        S[v][i4] =
            s_in != nullptr && sg == 0 ? s_in[((size_t)seq * Hv + h) * hs + slice(v) + (size_t)i4 * DK] : 0.f;
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // settle the state loads before the pipelined loop

  TOut* out = trans ? reinterpret_cast<TOut*>(seg.trans_out) : o;
  a.flags = nullptr;
  a.flag_step = 0;
  a.spin_max = 0;
  if (wave < 4)
    state_loop<true, TOut, false, NV>(sh, a, out, S);
  else
    state_loop<false, TOut, false, NV>(sh, a, out, S);

  if (trans) {  // the segment map transposed (M^T[n][k] = M[k][n]), as bf16 hi and lo parts [K][K] each
    uint16_t* mt = reinterpret_cast<uint16_t*>(seg.trans_final + ((size_t)run * Hv + h) * hs);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const size_t off = mt_frag(ncol, (vb + v) * VB + 4 * (l >> 4));
      uint32_t h01, l01, h23, l23;
      split2(S[v][0], S[v][1], h01, l01);
      split2(S[v][2], S[v][3], h23, l23);
      *reinterpret_cast<uint2*>(mt + off) = make_uint2(h01, h23);
      *reinterpret_cast<uint2*>(mt + hs + off) = make_uint2(l01, l23);
    }
    return;
  }
  float* fin = seg.G > 1 ? seg.local_final + ((size_t)run * Hv + h) * hs
                         : s_out != nullptr ? s_out + ((size_t)seq * Hv + h) * hs : nullptr;
  if (fin != nullptr) {
#pragma unroll
    for (int v = 0; v < NV; ++v)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) fin[slice(v) + (size_t)i4 * DK] = S[v][i4];
  }
}

// ------------------------------------------------------------------------------- phases 1 and 2 overlapped
//
// One launch in which phase 1 and the state pass run side by side. The state pass of a (sequence, head) chain
// starts once phase 1 has stored the chain's first chunk and then trails it, instead of waiting for every item
// of every chain: for few chains (unpacked batches of 8 .. 32 at 8 XCDs) part of phase 1 hides under the
// state pass, which holds one CU per 16 value rows of each chain; for many chains (packed batches) the state
// jobs of early chains run while phase 1 works on later ones. (The bytes moved stay the same: the workspace
// still goes to memory and back.) Where this pays is measured, see overlap_wanted.
//
// Producer and consumers of a chunk's workspace must share one L2: the XCDs' L2 caches are not coherent with
// each other, and the fences that would make them so write back or drop a whole L2. So every chain belongs to
// one queue, chain % n_q, and a workgroup serves the queue of the XCD it runs on (the hardware XCC_ID
// register). Each workgroup takes one role when it arrives: state worker or item worker. Item workers take the
// queue's items from an item ticket in a fixed order until none are left; state workers take its state jobs
// (chain x 8 value blocks, chains in queue order) from a state ticket. An item's workgroup sets the item's
// ready flag once its workspace stores have reached the L2; a state job reads each chunk's flag (one chunk
// ahead) before its loads. No data of a chunk is in any L1 before its flag is set (only state jobs read the
// workspace, and only after the flag), so plain loads see the stores through the shared L2.
// Roles go by placement, not by arrival order: the queue's first arrival takes items; a later workgroup takes
// a state role if it is the first to arrive on its CU (per-CU arrival count, keyed by XCC_ID and the HW_ID
// register's shader engine, array and CU) and the queue's state roles (8 nch for few chains, FQ_STATE_WORKERS
// for many) are not all taken; every other workgroup takes items. The dispatcher puts workgroups b and
// b + n_cu on one CU and arrivals only roughly follow blockIdx, so roles by arrival put two state workgroups on
// one CU now and then; the second then finished its chain 20-30 us after every other (T = 4096, 16 heads:
// the kernel's 82-99 us against 71-76 us for the rest).
//   few chains (at most FQ_FEW_CHAINS a queue, unpacked): one state job each; items in chunk order across the
//     queue's chains.
//   many chains: state jobs one after another; items chain after chain, so state jobs start in the order
//     their chains are produced.
// Progress: items never wait and every queue's first arrival takes items, so every item is stored whatever the
// number of resident workgroups; the queue's second arrival is the first to claim its CU (the first arrival
// claims none), so every queue of two or more workgroups (the grid gives each about 2 per CU of its XCD) has a
// state worker, and state workers take jobs until none are left. A wait that runs out (the spin bound) sets the
// device status word and the kernel still ends.
// The control block (per-queue tickets, per-CU arrival counts, one flag per item) is zeroed before each launch.
constexpr int FQ_MAX = 8;              // queues (one per XCD)
constexpr int FQ_FEW_CHAINS = 4;       // chains per queue of the few-chains order (32 state workgroups of 64)
constexpr int FQ_STATE_WORKERS = 24;   // workgroups per queue taking state jobs in the many-chains order
constexpr int FQ_MAX_SEQS = 256;       // packed sequences (LDS table of chunk offsets)
constexpr int FQ_MAX_QCHAINS = 512;    // chains per queue in the many-chains order (LDS table)

struct FusedCtl {
  // queue q: role ticket at [96 q], state-role count at [96 q + 16], item ticket at [96 q + 32], state
  // ticket at [96 q + 64]
  int* tickets;
  int* cu_claims;  // [FQ_CU_KEYS]: arrivals per CU (key of cu_key)
  int* flags;      // [n_items]
  int n_q;       // queues in use (XCDs of the device)
  int few;       // few-chains order
  int spin_max;  // bound of each wait for a ready flag
  int never_ready;  // state jobs read a zero word in place of their flags (the wait's error path)
};

constexpr int FQ_ZERO_WORD = 96 * FQ_MAX;  // the int after the tickets: zeroed with the block, never written
constexpr int FQ_CU_KEYS = 8 * 256;        // CU keys: XCD (3 bits) x shader engine, array, CU (HW_ID bits 15:8)
constexpr int FQ_CLAIMS = 832;             // int offset of the per-CU arrival counts (after 256 B of padding)
// tickets (8 queues x 3 lines of 128 bytes), the zero word and padding, the per-CU arrival counts
constexpr size_t FQ_HEADER = 4 * ((size_t)FQ_CLAIMS + FQ_CU_KEYS);
static_assert(FQ_HEADER % 256 == 0 && FQ_ZERO_WORD < FQ_CLAIMS, "control block layout");
size_t fused_ctl_bytes(int n_items) { return FQ_HEADER + (((size_t)n_items * 4 + 255) / 256) * 256; }

__global__ void zero_ints_kernel(int* p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}

union FusedShared {
  PrepShared p;
  StateShared s;
};

// Exclusive prefix sum over the workgroup's threads (x of thread t at position t): out[t] for t < n, out[n] the
// total. wsum: 8 ints of LDS.
__device__ __forceinline__ void block_exclusive_scan(int x, int n, int* out, int* wsum) {
  const int l = lane_id(), w = threadIdx.x >> 6;
  int inc = x;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(inc, d);
    if (l >= d) inc += y;
  }
  if (l == 63) wsum[w] = inc;
  __syncthreads();
  int base = 0;
  for (int i = 0; i < w; ++i) base += wsum[i];
  if ((int)threadIdx.x < n) out[threadIdx.x] = base + inc - x;
  if ((int)threadIdx.x == n - 1) out[n] = base + inc;
  if (n == 0 && threadIdx.x == 0) out[0] = 0;
  __syncthreads();
}

template <typename TG, bool GATE>
__global__ __launch_bounds__(P1_THREADS, P1_WAVES_PER_SIMD) void chunk_fused_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const TG* __restrict__ g, const TG* __restrict__ beta, const float* __restrict__ A_log,
    const float* __restrict__ dt_bias, const int32_t* __restrict__ cu, const int32_t* __restrict__ chunk_idx,
    int n_seqs, int n_chunks, int T, int Hk, int Hv, float scale, int qk_l2norm, const RowStrides rs,
    uint8_t* ws, const float* __restrict__ s_in, float* __restrict__ s_out, bf16* __restrict__ o,
    const FusedCtl ctl) {
  __shared__ FusedShared sm;
  __shared__ int tk;
  __shared__ int wsum[8];
  __shared__ int seq_c0[FQ_MAX_SEQS + 1];   // packed: first chunk of each sequence
  __shared__ int qpref[FQ_MAX_QCHAINS + 1];  // many chains: first item ticket of each chain of the queue
  int xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(xcc));
  const int qi = xcc % ctl.n_q;
  const int nct_t = (T + CH - 1) / CH;  // unpacked: chunks per sequence
  const int n_chains = n_seqs * Hv;
  const int nch = (n_chains - qi + ctl.n_q - 1) / ctl.n_q;  // chains of this queue: qi + n_q m, m < nch
  const int n_state = nch * (DV / VB);
  const int n_items = n_chunks * Hv;
  auto seq_bos = [&](int sq) {
    if (cu == nullptr) return sq * T;
    int sb, se;
    seq_bounds(cu, sq, T, sb, se);
    return sb;
  };
  auto seq_len = [&](int sq) {
    if (cu == nullptr) return T;
    int sb, se;
    seq_bounds(cu, sq, T, sb, se);
    return se - sb;
  };

  // tables of the many-chains order
  if (!ctl.few) {
    if (cu != nullptr) {
      const int t = threadIdx.x;
      block_exclusive_scan(t < n_seqs ? (seq_len(t) + CH - 1) / CH : 0, n_seqs, seq_c0, wsum);
    }
    const int t = threadIdx.x;
    int len = 0;
    if (t < nch) {
      const int sq = (qi + ctl.n_q * t) / Hv;
      len = (seq_len(sq) + CH - 1) / CH;
    }
    block_exclusive_scan(len, nch, qpref, wsum);
  }
  auto chunk0 = [&](int sq) { return cu != nullptr ? seq_c0[sq] : sq * nct_t; };
  const int n_q_items = ctl.few ? nch * nct_t : qpref[nch];

  // role (state or items)
  const int n_workers = ctl.few ? n_state : min(n_state, FQ_STATE_WORKERS);
  if (threadIdx.x == 0) {
    int state = 0;
    if (__hip_atomic_fetch_add(ctl.tickets + 96 * qi, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) > 0) {
      unsigned hw;
      asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
      const int key = ((xcc & 7) << 8) | (int)((hw >> 8) & 0xff);  // XCD, shader engine, array, CU
      if (__hip_atomic_fetch_add(ctl.cu_claims + key, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0 &&
          __hip_atomic_fetch_add(ctl.tickets + 96 * qi + 16, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < n_workers)
        state = 1;
    }
    tk = state;
  }
  __syncthreads();

  if (tk != 0) {
    const int l = lane_id(), wave = threadIdx.x >> 6;
    __builtin_amdgcn_s_setprio(3);  // the sequential pass's waves issue ahead of phase-1 waves on their CU
    for (;;) {
      __syncthreads();  // every thread has read tk (and the LDS of the last job is free)
      if (threadIdx.x == 0)
        tk = __hip_atomic_fetch_add(ctl.tickets + 96 * qi + 64, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __syncthreads();
      const int js = tk;
      if (js >= n_state) break;
      const int ch = qi + ctl.n_q * (js / (DV / VB)), vb = js % (DV / VB);
      const int sq = ch / Hv, h = ch % Hv;
      StateArgs a;
      a.ws = ws;
      a.Hv = Hv;
      a.h = h;
      a.vb = vb;
      a.xs = 1.f;
      a.bos = seq_bos(sq);
      a.len = seq_len(sq);
      a.c0 = chunk0(sq);
      a.nchunks = max(0, min((a.len + CH - 1) / CH, n_chunks - a.c0));
      // (never_ready: the job reads the zero word in place of its flags; applying the test to the flag values
      // instead puts a wait for each prefetched flag right behind its load)
      a.flags = ctl.never_ready ? ctl.tickets + FQ_ZERO_WORD : ctl.flags + (size_t)a.c0 * Hv + h;
      a.flag_step = ctl.never_ready ? 0 : Hv;
      a.spin_max = ctl.spin_max;
      const int ncol = 16 * wave + (l & 15);
      const size_t slice = ((size_t)vb * VB + 4 * (l >> 4)) * DK + ncol;
      const size_t hs = (size_t)DV * DK;
      f32x4 S[1];
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4)
        S[0][i4] = s_in != nullptr ? s_in[((size_t)sq * Hv + h) * hs + slice + (size_t)i4 * DK] : 0.f;
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      if (wave < 4)
        state_loop<true, bf16, true, 1>(sm.s, a, o, S);
      else
        state_loop<false, bf16, true, 1>(sm.s, a, o, S);
      if (s_out != nullptr) {
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) s_out[((size_t)sq * Hv + h) * hs + slice + (size_t)i4 * DK] = S[0][i4];
      }
    }
    return;
  }

  // item workers: ticket u of the queue -> item (chunk x head); thread 0 decodes it for the workgroup
  auto item_of = [&](int u) {
    int m, c;
    if (ctl.few) {  // chunk order across the chains: u = chunk * nch + m
      m = u % nch;
      c = u / nch;
    } else {  // chain after chain: the last chain m with qpref[m] <= u
      int lo = 0, hi = nch - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (qpref[mid] <= u) lo = mid;
        else hi = mid - 1;
      }
      m = lo;
      c = u - qpref[m];
    }
    const int ch = qi + ctl.n_q * m;
    return (chunk0(ch / Hv) + c) * Hv + ch % Hv;
  };
  auto take = [&]() {  // thread 0: the queue's next item (-1: none left)
    const int u = __hip_atomic_fetch_add(ctl.tickets + 96 * qi + 32, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return u < n_q_items ? item_of(u) : -1;
  };
  // the next ticket is taken as an item starts and its rows load while the item computes (items past a short
  // chunk table, >= n_items, have no workspace and are passed over)
  prep_init(sm.p.b);
  const PrepLane L(lane_id());
  const PrepRows lr(threadIdx.x, rs);
  RowRegs R;
  if (threadIdx.x == 0) tk = take();
  __syncthreads();
  int cur = tk;
  __syncthreads();  // every thread has read tk
  if (cur >= 0 && cur < n_items)
    load_rows<P1_WAVES>(R, item_at(cur, cu, chunk_idx, n_seqs, T, Hk, Hv), q, k, v, rs, lr.oq, lr.ok, lr.ov);
  while (cur >= 0) {
    if (threadIdx.x == 0) tk = take();
    __syncthreads();  // tk visible (and the LDS of the last item is free)
    const int nxt = tk;
    const int nload = nxt >= 0 && nxt < n_items ? nxt : -1;
    if (cur < n_items) {
      const ItemAt ic = item_at(cur, cu, chunk_idx, n_seqs, T, Hk, Hv);
      const ItemAt in = item_at(nload >= 0 ? nload : cur, cu, chunk_idx, n_seqs, T, Hk, Hv);
      prep_item<TG, GATE, false, P1_WAVES>(sm.p.b, ic, R, nload >= 0, in, q, k, v, g, beta, A_log, dt_bias, Hv, scale, qk_l2norm, rs,
                          ws, L, lr.rowoff, lr.oq, lr.ok, lr.ov);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's workspace stores are in the L2
      __syncthreads();
      if (threadIdx.x == 0) __hip_atomic_store(ctl.flags + cur, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      if (nload >= 0)
        load_rows<P1_WAVES>(R, item_at(nload, cu, chunk_idx, n_seqs, T, Hk, Hv), q, k, v, rs, lr.oq, lr.ok, lr.ov);
      __syncthreads();  // every thread has read tk
    }
    cur = nxt;
  }
}

// S_g for the segments g >= 1 of one (sequence, head), as bf16 [V][K] for the correction, and the final
// state: S_1 = L_0, S_{g+1} = S_g M_g + L_g, final = S_{G-1} M_{G-1} + L_{G-1}. Rows of S never mix (M acts
// from the right), so each workgroup carries 16 rows through the whole chain on its own: 8 workgroups per
// (sequence, head). Its rows sit in LDS as bf16 hi and lo parts; each of the 4 waves forms 32 columns of the
// product on bf16 MFMA (S_hi M_hi + S_hi M_lo + S_lo M_hi: about 16 significant bits, the fp32 state's
// accuracy) with M^T's hi and lo rows, as the state pass stored them, read straight from memory. The chain is
// bound by those reads (64 KiB a step for every workgroup, about 2 us): each step's are issued during the
// previous step's products.
constexpr int CB_ROWS = 16, CB_LDH = DK + 8, CB_LDT = DK + 4;

__global__ __launch_bounds__(256) void chunk_combine_kernel(const float* __restrict__ local_final,
                                                            const float* __restrict__ trans_final_t,
                                                            uint16_t* __restrict__ s_start,
                                                            float* __restrict__ s_out, int Hv, int G) {
  __shared__ uint16_t Shi[CB_ROWS][CB_LDH], Slo[CB_ROWS][CB_LDH];  // A operands (bf16 hi / lo of S)
  __shared__ float Tmp[CB_ROWS][CB_LDT];                            // S M_g, fp32
  const int rb = blockIdx.x % (DV / CB_ROWS), pair = blockIdx.x / (DV / CB_ROWS);
  const int seq = pair / Hv, h = pair % Hv, r0 = rb * CB_ROWS;
  const int tid = threadIdx.x, l = tid & 63, wave = tid >> 6;
  const int er = tid >> 4, ec = (tid & 15) * 8;  // this thread's 8 elements of the 16 rows
  const size_t hs = (size_t)DV * DK;
  auto L = [&](int g) { return local_final + (((size_t)seq * G + g) * Hv + h) * hs + (size_t)(r0 + er) * DK + ec; };
  auto MT = [&](int g) {
    return reinterpret_cast<const uint16_t*>(trans_final_t + (((size_t)seq * (G - 1) + g - 1) * Hv + h) * hs);
  };
  const bool want_final = s_out != nullptr;
  auto needed = [&](int g) { return g < G - 1 || (g == G - 1 && want_final); };  // step g's product
  // B fragments of column tile t (M^T rows 32 wave + 16 t + l % 16) and key block k (32 k + 8 (l / 16) ..),
  // stored in fragment order (mt_frag): 1 KiB of contiguous memory per load
  auto load_b = [&](const uint16_t* mt, int k, uint4* b) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const uint16_t* p = mt + mt_frag(32 * wave + 16 * t + (l & 15), 32 * k + 8 * (l >> 4));
      b[(t * (DK / 32) + k) * 2] = *reinterpret_cast<const uint4*>(p);
      b[(t * (DK / 32) + k) * 2 + 1] = *reinterpret_cast<const uint4*>(p + hs);
    }
  };
  auto load_l = [&](int g, float4* v) {
    v[0] = *reinterpret_cast<const float4*>(L(g));
    v[1] = *reinterpret_cast<const float4*>(L(g) + 4);
  };
  auto put_s = [&](float4 a, float4 b) {  // 8 elements into the hi / lo tiles
    uint32_t hw[4], lw[4];
    split2(a.x, a.y, hw[0], lw[0]);
    split2(a.z, a.w, hw[1], lw[1]);
    split2(b.x, b.y, hw[2], lw[2]);
    split2(b.z, b.w, hw[3], lw[3]);
    *reinterpret_cast<uint4*>(&Shi[er][ec]) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    *reinterpret_cast<uint4*>(&Slo[er][ec]) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
  };
  constexpr int NB = 2 * (DK / 32) * 2;
  float4 l0[2], l1[2];
  uint4 b0[NB], b1[NB];
  load_l(0, l0);
  put_s(l0[0], l0[1]);  // S_1 = L_0
  if (needed(1)) {
#pragma unroll
    for (int k = 0; k < DK / 32; ++k) load_b(MT(1), k, b0);
    load_l(1, l0);
  }
  // one step: S_g out as bf16, then S <- S M_g + L_g from (bv, lv); the next step's operands into (bn, ln)
  auto step = [&](int g, const uint4* bv, const float4* lv, uint4* bn, float4* ln) __attribute__((always_inline)) {
    const bool pre = needed(g + 1);
    __syncthreads();  // the hi / lo tiles hold S_g
    uint16_t* so = s_start + (((size_t)seq * (G - 1) + g - 1) * Hv + h) * hs + (size_t)(r0 + er) * DK + ec;
    *reinterpret_cast<uint4*>(so) = *reinterpret_cast<const uint4*>(&Shi[er][ec]);  // bf16 S_g = its hi part
    if (!needed(g)) return;  // the last segment, the final state not wanted
    if (pre) load_l(g + 1, ln);
    f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int k = 0; k < DK / 32; ++k) {
      if (pre) load_b(MT(g + 1), k, bn);
      const bf16x8 ah = *reinterpret_cast<const bf16x8*>(&Shi[l & 15][32 * k + 8 * (l >> 4)]);
      const bf16x8 al = *reinterpret_cast<const bf16x8*>(&Slo[l & 15][32 * k + 8 * (l >> 4)]);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const bf16x8 bh = __builtin_bit_cast(bf16x8, bv[(t * (DK / 32) + k) * 2]);
        const bf16x8 bl = __builtin_bit_cast(bf16x8, bv[(t * (DK / 32) + k) * 2 + 1]);
        acc[t] = mfma(ah, bh, acc[t]);
        acc[t] = mfma(ah, bl, acc[t]);
        acc[t] = mfma(al, bh, acc[t]);
      }
    }
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) Tmp[4 * (l >> 4) + i][32 * wave + 16 * t + (l & 15)] = acc[t][i];
    __syncthreads();  // every wave has read the hi / lo tiles and written its columns of S M_g
    const float4 p0 = *reinterpret_cast<const float4*>(&Tmp[er][ec]);
    const float4 p1 = *reinterpret_cast<const float4*>(&Tmp[er][ec + 4]);
    const float4 s0 = make_float4(p0.x + lv[0].x, p0.y + lv[0].y, p0.z + lv[0].z, p0.w + lv[0].w);
    const float4 s1 = make_float4(p1.x + lv[1].x, p1.y + lv[1].y, p1.z + lv[1].z, p1.w + lv[1].w);
    if (g == G - 1) {  // the final state, fp32
      float* fo = s_out + ((size_t)seq * Hv + h) * hs + (size_t)(r0 + er) * DK + ec;
      *reinterpret_cast<float4*>(fo) = s0;
      *reinterpret_cast<float4*>(fo + 4) = s1;
    } else {
      put_s(s0, s1);
    }
  };
  for (int g = 1; g < G; g += 2) {
    step(g, b0, l0, b1, l1);
    if (g + 1 < G) step(g + 1, b1, l1, b0, l0);
  }
}

// o[t][h][:] += (Q' P^T)[t][h][:] S_g^T for the rows of one chunk of a segment g >= 1: D = S_g . (Q'P^T)^T on
// bf16 MFMA with the values as the M side (A = S_g rows, staged once in LDS for the 4 waves) and the tokens as
// the N side (B = Q'P^T rows), so each lane's D values are 4 adjacent values of one row of o (one 8-byte
// read-modify-write, its read issued first). 4 waves x 16 tokens.
constexpr int CR_LD = DK + 8;  // bf16 row stride of the staged S_g: 272 bytes, rows 4 banks apart
template <typename TOut>
__global__ __launch_bounds__(256) void chunk_correct_kernel(const uint16_t* __restrict__ s_start,
                                                            const uint16_t* __restrict__ trans_out,
                                                            TOut* __restrict__ o, int T, int Hv, int G, int Cs) {
  __shared__ uint16_t Ssh[DV][CR_LD];
  using OWord = std::conditional_t<sizeof(TOut) == 2, uint2, float4>;  // 4 outputs
  const int nseg = G - 1;
  const int c = blockIdx.x % Cs, h = (blockIdx.x / Cs) % Hv, run = blockIdx.x / (Cs * Hv);
  const int seq = run / nseg, sg = 1 + run % nseg;
  const int t0 = sg * Cs * CH + c * CH;  // within the sequence
  if (t0 >= T) return;                   // the whole workgroup
  const int len = min(CH, T - t0);
  const int tid = threadIdx.x, l = tid & 63, wave = tid >> 6;
  const int tok = 16 * wave + (l & 15);
  const bool live = tok < len;
  const uint16_t* S = s_start + (((size_t)seq * nseg + sg - 1) * Hv + h) * (size_t)DV * DK;
  const size_t row0 = (size_t)seq * T + t0;
  TOut* orow = o + ((row0 + tok) * Hv + h) * DV + 4 * (l >> 4);
  OWord ow[DV / 16];
  uint4 bw[DK / 32];
  if (live) {
#pragma unroll
    for (int t = 0; t < DV / 16; ++t) ow[t] = *reinterpret_cast<const OWord*>(orow + 16 * t);
#pragma unroll
    for (int kq = 0; kq < DK / 32; ++kq)
      bw[kq] = *reinterpret_cast<const uint4*>(trans_out + ((row0 + tok) * Hv + h) * DK + 32 * kq + 8 * (l >> 4));
  } else {
#pragma unroll
    for (int kq = 0; kq < DK / 32; ++kq) bw[kq] = make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < DV * DK / 8 / 256; ++i) {  // S_g -> LDS, 16 bytes a thread per pass
    const int e = tid + 256 * i, r = e / (DK / 8), c8 = (e % (DK / 8)) * 8;
    *reinterpret_cast<uint4*>(&Ssh[r][c8]) = *reinterpret_cast<const uint4*>(S + (size_t)r * DK + c8);
  }
  __syncthreads();
  f32x4 acc[DV / 16];
#pragma unroll
  for (int t = 0; t < DV / 16; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kq = 0; kq < DK / 32; ++kq) {
    const bf16x8 b = __builtin_bit_cast(bf16x8, bw[kq]);
#pragma unroll
    for (int t = 0; t < DV / 16; ++t) {
      const bf16x8 a = *reinterpret_cast<const bf16x8*>(&Ssh[16 * t + (l & 15)][32 * kq + 8 * (l >> 4)]);
      acc[t] = mfma(a, b, acc[t]);
    }
  }
  if (!live) return;
#pragma unroll
  for (int t = 0; t < DV / 16; ++t) {
    if constexpr (sizeof(TOut) == 2) {
      const uint2 w = ow[t];
      const float v0 = __uint_as_float(w.x << 16) + acc[t][0], v1 = __uint_as_float(w.x & 0xffff0000u) + acc[t][1];
      const float v2 = __uint_as_float(w.y << 16) + acc[t][2], v3 = __uint_as_float(w.y & 0xffff0000u) + acc[t][3];
      *reinterpret_cast<uint2*>(orow + 16 * t) = make_uint2(pack_bf16x2(v0, v1), pack_bf16x2(v2, v3));
    } else {
      const float4 w = ow[t];
      *reinterpret_cast<float4*>(orow + 16 * t) =
          make_float4(w.x + acc[t][0], w.y + acc[t][1], w.z + acc[t][2], w.w + acc[t][3]);
    }
  }
}

// Segments for an unpacked batch of B sequences of T tokens (G == 1: the plain pass). Costs measured on
// MI355X at 4 heads, one sequence (graph replay, hundredths of a microsecond): the plain pass 64 a chunk; a
// segmented one 80 a chunk of a segment, 207 a combine step and 985 fixed (the combine's and the correction's
// launches and the longer state pass). A segment count in 2 .. 8 is taken when its local and transition
// workgroups all fit one per CU and it is the cheapest.
// NV: value blocks of 16 rows per state-pass workgroup. Two when the plain pass's workgroups of one block
// would outnumber the CUs (more than n_cu / 8 chains): each then reads a chunk's shared operands (W' or Q',
// K^T) once for 32 value rows, and the pass needs half the workgroup slots, for chunk steps about 1.4x as long
// (measured: 32 packed sequences of 30,526 tokens at 16 heads, 4,096 one-block workgroups, 506 us with two
// blocks against 552; one 4096-token sequence at 16 heads, 128 workgroups, 92.5 us with two against 73.6).
struct SegPlan {
  int G, Cs;
  int NV;
};
int state_nv(long chains, int n_cu) { return chains * (DV / VB) > n_cu ? 2 : 1; }
SegPlan seg_plan(int B, int T, int Hv, int n_cu) {
  const int nct = (T + CH - 1) / CH;
  const long base = (long)B * Hv * (DV / VB);
  SegPlan p{1, nct, state_nv((long)B * Hv, n_cu)};
  if (nct < 8 || 2 * base > n_cu) return p;  // (a segment holds at least 4 chunks)
  long best = 64L * nct;
  for (int g = 2; g <= 8; ++g) {
    const int cs = (nct + g - 1) / g, gg = (nct + cs - 1) / cs;
    if (cs < 4 || gg < 2 || base * (2 * gg - 1) > n_cu) continue;
    const long cost = 985 + 80L * cs + 207L * (gg - 1);
    if (cost < best) {
      best = cost;
      p = SegPlan{gg, cs, 1};
    }
  }
  return p;
}

// Bytes past the phase-1 workspace a segmented run needs: Q'P^T (bf16 [B*T][Hv][K]), L (fp32, G per
// sequence), M^T (bf16 hi and lo, G - 1 per sequence), S_g (bf16, G - 1 per sequence).
size_t seg_bytes(int B, int T, int Hv, const SegPlan& p) {
  if (p.G <= 1) return 0;
  const size_t hs = (size_t)DV * DK;
  return (size_t)B * T * Hv * DK * 2 + (size_t)B * Hv * hs * (4 * p.G + 4 * (p.G - 1) + 2 * (p.G - 1));
}

// Launch form of the chunked path: -1 the library's choice, 0 always two launches, 1 the overlapped launch for
// every eligible batch. Set by zgdn_chunk_set_launch_form; its initial value comes from ZGDN_CHUNK_OVERLAP
// ("0" / "1"), read once when the library is loaded, so that no call reads the environment.
int launch_form_from_env() {
  const char* e = std::getenv("ZGDN_CHUNK_OVERLAP");
  if (e != nullptr && e[0] == '0') return 0;
  if (e != nullptr && e[0] == '1') return 1;
  return -1;
}
std::atomic<int> g_launch_form{launch_form_from_env()};

// Spin bound of the overlapped launch's waits and the never-ready test switch (zgdn_chunk_set_wait_limit).
std::atomic<int> g_spin_max{SPIN_MAX};
std::atomic<int> g_never_ready{0};

// Whether an eligible batch takes the overlapped launch: only when the launch form asks for it. With the
// phase-1 item of this file the two launches measured faster on every shape tried (MI355X, bf16,
// dk = dv = 128, HIP graph replay, us two launches / overlapped, both forms forced in one process):
// 1 x 4096 at 16 heads 81.3 / 86.4, at 8 heads 57.3 / 57.7; 2 x 4096 139.6 / 168.0; 1 x 2048 47.2 / 56.3;
// 4 x 1024 63.9 / 81.7; packed 32 x 512, 16 x 1024, 8 x 2048 310.2 / 347.3, 303.6 / 312.7, 302.6 / 311.8;
// 32 packed sequences of 64 .. 2048 tokens 730.0 / 747.7. (The overlapped launch won where phase 1 was slower:
// with an item of 10-11k VALU instructions it took the 4096-token, 16-head prefill in 78-81 us against 83 us,
// and the 32-sequence packed batch in 548-559 against 624-634 us.) The overlapped state jobs share their CUs
// with phase-1 workgroups, which slows their chunk steps by a third, and the faster phase 1 leaves less of its
// time to hide.
bool overlap_wanted(bool, long, double, long) { return g_launch_form.load(std::memory_order_relaxed) == 1; }

int device_cus() {
  int dev = 0, n_cu = 256;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    n_cu = 256;
  return std::max(1, n_cu);
}

// Queues of the overlapped launch: one per XCD (their L2s are not coherent with each other), or 0 when the
// device's shape does not allow the launch (an XCD count the control block has no room for, or CUs that do
// not split evenly over the XCDs, so that the XCC_ID register would not name one queue per L2).
int overlap_queues(int n_cu, int n_xcc) {
  if (n_xcc < 1 || n_xcc > FQ_MAX || n_cu < n_xcc || n_cu % n_xcc != 0) return 0;
  return n_xcc;
}

int device_xccs() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess)
    return 0;
  return n;
}

template <typename TG>
void launch_prep(bool gate, int nchunks, int Hk, int Hv, const void* q, const void* k, const void* v, const void* g,
                 const void* beta, const float* A_log, const float* dt_bias, const int32_t* cu,
                 const int32_t* chunk_idx, int n_seqs, int T, float scale, int qk_l2norm, const RowStrides& rs,
                 uint8_t* ws, hipStream_t stream) {
  // P1_WGS_PER_CU resident workgroups per CU (what the LDS footprint allows), each looping over items
  int dev = 0, n_cu = 256;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    n_cu = 256;
  const int n_items = nchunks * Hv;
  // at most one item a CU: one workgroup of 16 waves each (the item's latency is the phase's time)
  const bool wide = n_items <= std::max(1, n_cu);
  const dim3 grid(wide ? n_items : std::min(n_items, P1_WGS_PER_CU * std::max(1, n_cu)));
#define ZGDN_PREP(GT, WV)                                                                                          \
  hipLaunchKernelGGL((chunk_prep_kernel<TG, GT, WV>), grid, dim3(64 * (WV)), 0, stream, (const uint16_t*)q,       \
                     (const uint16_t*)k, (const uint16_t*)v, (const TG*)g, (const TG*)beta, A_log, dt_bias, cu,    \
                     chunk_idx, n_seqs, n_items, T, Hk, Hv, scale, qk_l2norm, rs, ws)
  if (gate) {
    if (wide) ZGDN_PREP(true, 16);
    else ZGDN_PREP(true, 8);
  } else {
    if (wide) ZGDN_PREP(false, 16);
    else ZGDN_PREP(false, 8);
  }
#undef ZGDN_PREP
}

}  // namespace
}  // namespace zgdn

extern "C" int zgdn_chunk_set_launch_form(int form) {
  if (form < -1 || form > 1) return zgdn::fail(ZGDN_EINVAL, "zgdn_chunk_set_launch_form: form %d (-1, 0 or 1)", form);
  zgdn::g_launch_form.store(form);
  return ZGDN_OK;
}

extern "C" int zgdn_chunk_get_launch_form(void) { return zgdn::g_launch_form.load(); }

extern "C" int zgdn_chunk_set_wait_limit(int spins, int never_ready) {
  if (spins < 0) return zgdn::fail(ZGDN_EINVAL, "zgdn_chunk_set_wait_limit: spins %d", spins);
  zgdn::g_spin_max.store(spins == 0 ? zgdn::SPIN_MAX : spins);
  zgdn::g_never_ready.store(never_ready != 0);
  return ZGDN_OK;
}

extern "C" int zgdn_chunk_status(int* status, int clear) {
  if (status == nullptr) return zgdn::fail(ZGDN_EINVAL, "zgdn_chunk_status: null pointer");
  *status = 0;
  hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemcpyFromSymbol(status, HIP_SYMBOL(zgdn::g_chunk_status), sizeof(int));
  if (e == hipSuccess && clear) {
    const int zero = 0;
    e = hipMemcpyToSymbol(HIP_SYMBOL(zgdn::g_chunk_status), &zero, sizeof(int));
  }
  if (e != hipSuccess) return zgdn::fail(ZGDN_EHIP, "zgdn_chunk_status: %s", hipGetErrorString(e));
  return ZGDN_OK;
}

extern "C" int zgdn_chunk_status_async(int* host_status, void* stream) {
  if (host_status == nullptr) return zgdn::fail(ZGDN_EINVAL, "zgdn_chunk_status_async: null pointer");
  const hipError_t e = hipMemcpyFromSymbolAsync(host_status, HIP_SYMBOL(zgdn::g_chunk_status), sizeof(int), 0,
                                                hipMemcpyDeviceToHost, (hipStream_t)stream);
  if (e != hipSuccess) return zgdn::fail(ZGDN_EHIP, "zgdn_chunk_status_async: %s", hipGetErrorString(e));
  return ZGDN_OK;
}

extern "C" int zgdn_chunk_overlap_queues(int n_cu, int n_xcc) { return zgdn::overlap_queues(n_cu, n_xcc); }

extern "C" size_t zgdn_chunk_workspace_size(int n_chunks, int Hv) {
  const size_t items = (size_t)(n_chunks > 0 ? n_chunks : 0) * (size_t)(Hv > 0 ? Hv : 0);
  return items * zgdn::WS_CHUNK + zgdn::fused_ctl_bytes((int)items);
}

extern "C" size_t zgdn_chunk_workspace_bytes(int n_chunks, int Hv, int K, int V, int qkv_dtype) {
  if (K != V || (K != 64 && K != 128) || (qkv_dtype != ZGDN_F32 && qkv_dtype != ZGDN_BF16)) return 0;
  if (qkv_dtype == ZGDN_BF16 && K == zgdn::DK) return zgdn_chunk_workspace_size(n_chunks, Hv);
  const size_t items = (size_t)(n_chunks > 0 ? n_chunks : 0) * (size_t)(Hv > 0 ? Hv : 0);
  return items * zgdn::chunk32_item_bytes(K);
}

extern "C" size_t zgdn_chunk_segment_workspace_size(int B, int T, int Hv) {
  using namespace zgdn;
  if (B < 1 || T < 1 || Hv < 1) return 0;
  return seg_bytes(B, T, Hv, seg_plan(B, T, Hv, device_cus()));
}

namespace zgdn {
namespace {
// The chunked forward behind zgdn_chunk_fwd and zgdn_chunk_fwd_noalloc (`fn` names the entry in messages).
int chunk_fwd_impl(const char* fn, const void* q, const void* k, const void* v, int qkv_dtype, const void* g,
                   const void* beta, int gb_dtype, const float* A_log, const float* dt_bias, int qk_l2norm,
                   const float* initial_state, float* final_state, void* o, const int32_t* cu_seqlens,
                   const int32_t* chunk_indices, int n_seqs, int n_chunks, int B, int T, int Hk, int Hv, int K,
                   int V, long q_ld, long k_ld, long v_ld, long gb_ld, int beta_sigmoid, float scale,
                   void* workspace, size_t workspace_bytes, void* stream) {
  // (with no tokens, T == 0, the token arrays may be empty allocations: only the states are touched)
  if (!workspace || (T > 0 && (!q || !k || !v || !g || !beta || !o)))
    return fail(ZGDN_EINVAL, "%s: null pointer", fn);
  if (qkv_dtype != ZGDN_F32 && qkv_dtype != ZGDN_BF16) return fail(ZGDN_EINVAL, "%s: dtype code %d", fn, qkv_dtype);
  if (K != V || (K != 64 && K != 128))
    return fail(ZGDN_EUNSUPPORTED, "%s: K=%d V=%d (supported: K == V, 64 or 128)", fn, K, V);
  // bf16 q/k/v with 128-wide heads run on bf16 MFMA (this file); fp32 inputs and 64-wide heads on the
  // fp32-arithmetic path (gdn_chunk_f32.hip)
  const bool bf16_path = qkv_dtype == ZGDN_BF16 && K == DK;
  if (gb_dtype != ZGDN_F32 && gb_dtype != ZGDN_BF16) return fail(ZGDN_EINVAL, "%s: dtype code %d", fn, gb_dtype);
  if (B < 1 || T < 0 || Hk < 1 || Hv < 1 || Hv % Hk)
    return fail(ZGDN_EINVAL, "%s: bad sizes B=%d T=%d Hk=%d Hv=%d", fn, B, T, Hk, Hv);
  if ((A_log == nullptr) != (dt_bias == nullptr))
    return fail(ZGDN_EINVAL, "%s: A_log and dt_bias go together", fn);
  // row strides: at least a token's heads; q / k / v rows start on 16-byte boundaries (the kernels read
  // 16-byte groups: 8 bf16 or 4 fp32 elements)
  const long ve = qkv_dtype == ZGDN_F32 ? 4 : 8;
  if (q_ld < (long)Hk * K || k_ld < (long)Hk * K || v_ld < (long)Hv * V || gb_ld < Hv || q_ld % ve ||
      k_ld % ve || v_ld % ve || ((uintptr_t)q | (uintptr_t)k | (uintptr_t)v) % 16)
    return fail(ZGDN_EINVAL, "%s: row strides q=%ld k=%ld v=%ld g/beta=%ld (need >= a token's heads, q/k/v "
                "multiples of %ld elements from 16-byte aligned bases)", fn, q_ld, k_ld, v_ld, gb_ld, ve);
  const RowStrides rs{q_ld, k_ld, v_ld, gb_ld, beta_sigmoid != 0};
  int N = B;
  if (cu_seqlens != nullptr) {
    if (B != 1 || chunk_indices == nullptr || n_seqs < 1)
      return fail(ZGDN_EINVAL, "%s: packed sequences need B == 1, chunk_indices and n_seqs >= 1", fn);
    N = n_seqs;
  } else {
    n_chunks = B * ((T + CH - 1) / CH);
  }
  if (n_chunks < 0) return fail(ZGDN_EINVAL, "%s: n_chunks=%d", fn, n_chunks);
  const size_t need = zgdn_chunk_workspace_bytes(n_chunks, Hv, K, V, qkv_dtype);
  if (workspace_bytes < need)
    return fail(ZGDN_EINVAL, "%s: workspace of %zu bytes, need %zu", fn, workspace_bytes, need);
  hipStream_t s = (hipStream_t)stream;
  if (!bf16_path)
    return chunk32_fwd(fn, q, k, v, qkv_dtype, g, beta, gb_dtype, A_log, dt_bias, qk_l2norm, initial_state,
                       final_state, o, cu_seqlens, chunk_indices, N, n_chunks, T, Hk, Hv, K, scale, rs, workspace, s);
  uint8_t* ws = (uint8_t*)workspace;
  const bool gate = A_log != nullptr;
  // phase 2: plain runs, or (unpacked batches that would hold few CUs, workspace permitting) segmented runs
  const SegPlan plan =
      cu_seqlens == nullptr ? seg_plan(B, T, Hv, device_cus()) : SegPlan{1, 0, state_nv((long)N * Hv, device_cus())};
  const size_t base = zgdn_chunk_workspace_size(n_chunks, Hv);
  const bool segmented = plan.G > 1 && workspace_bytes >= base + seg_bytes(B, T, Hv, plan);
  SegRun run{1, (T + CH - 1) / CH, nullptr, nullptr, nullptr};
  uint16_t* s_start = nullptr;
  if (segmented) {
    const size_t hs = (size_t)DV * DK;
    uint8_t* p = ws + base;
    run.G = plan.G;
    run.Cs = plan.Cs;
    run.trans_out = reinterpret_cast<uint16_t*>(p);
    p += (size_t)B * T * Hv * DK * 2;
    run.local_final = reinterpret_cast<float*>(p);
    p += (size_t)B * plan.G * Hv * hs * 4;
    run.trans_final = reinterpret_cast<float*>(p);
    p += (size_t)B * (plan.G - 1) * Hv * hs * 4;
    s_start = reinterpret_cast<uint16_t*>(p);
  }
  // phases 1 and 2 in one overlapped launch where it pays (overlap_wanted): unpacked batches of 8 .. 16 long
  // chains (few-chains order) on the plain pass, packed batches of up to 256 sequences and unpacked batches of more
  // chains (many-chains order)
  const int n_q = overlap_queues(device_cus(), device_xccs());  // one queue per XCD; 0: no overlapped launch
  const long n_chains = (long)N * Hv;
  const bool few = cu_seqlens == nullptr && n_chains <= (long)FQ_FEW_CHAINS * n_q;
  const bool fits = n_q > 0 && (few || ((cu_seqlens == nullptr || N <= FQ_MAX_SEQS) &&
                                         (n_chains + n_q - 1) / n_q <= FQ_MAX_QCHAINS));
  if (!segmented && n_chunks > 0 && n_q > 0 && n_chains >= n_q && fits &&
      overlap_wanted(few, (long)n_chunks * Hv, (double)n_chunks / std::max(1, N), (n_chains + n_q - 1) / n_q)) {
    const int n_items = n_chunks * Hv;
    int* ctl_base = reinterpret_cast<int*>(ws + (size_t)n_items * WS_CHUNK);
    const FusedCtl ctl{ctl_base, ctl_base + FQ_CLAIMS, ctl_base + FQ_HEADER / 4, n_q, few ? 1 : 0,
                       g_spin_max.load(std::memory_order_relaxed), g_never_ready.load(std::memory_order_relaxed)};
    const int n_ctl = (int)(fused_ctl_bytes(n_items) / 4);
    hipLaunchKernelGGL(zero_ints_kernel, dim3((n_ctl + 255) / 256), dim3(256), 0, s, ctl_base, n_ctl);
    const dim3 grid(P1_WGS_PER_CU * device_cus());
#define ZGDN_FUSED(TGT, GT)                                                                                        \
  hipLaunchKernelGGL((chunk_fused_kernel<TGT, GT>), grid, dim3(P1_THREADS), 0, s, (const uint16_t*)q,             \
                     (const uint16_t*)k, (const uint16_t*)v, (const TGT*)g, (const TGT*)beta, A_log, dt_bias,    \
                     cu_seqlens, chunk_indices, N, n_chunks, T, Hk, Hv, scale, qk_l2norm, rs, ws, initial_state, \
                     final_state, (bf16*)o, ctl)
    if (gb_dtype == ZGDN_F32) {
      if (gate) ZGDN_FUSED(float, true);
      else ZGDN_FUSED(float, false);
    } else {
      if (gate) ZGDN_FUSED(bf16, true);
      else ZGDN_FUSED(bf16, false);
    }
#undef ZGDN_FUSED
    return check_launch(fn);
  }
  if (n_chunks > 0) {
    if (gb_dtype == ZGDN_F32)
      launch_prep<float>(gate, n_chunks, Hk, Hv, q, k, v, g, beta, A_log, dt_bias, cu_seqlens, chunk_indices,
                               N, T, scale, qk_l2norm, rs, ws, s);
    else
      launch_prep<bf16>(gate, n_chunks, Hk, Hv, q, k, v, g, beta, A_log, dt_bias, cu_seqlens, chunk_indices,
                              N, T, scale, qk_l2norm, rs, ws, s);
  }
  const long runs = (long)N * Hv * (2 * run.G - 1);  // local + transition (run, head) pairs
  // groups of 8 pairs x DV / VB / NV value-block groups
  const dim3 grid2((unsigned)(((runs + 7) / 8) * 8 * (DV / VB / plan.NV)));
  if (plan.NV == 2)
    hipLaunchKernelGGL((chunk_state_kernel<bf16, 2>), grid2, dim3(64 * P2_WAVES), 0, s, ws, initial_state,
                       final_state, (bf16*)o, cu_seqlens, N, n_chunks, T, Hv, run);
  else
    hipLaunchKernelGGL((chunk_state_kernel<bf16, 1>), grid2, dim3(64 * P2_WAVES), 0, s, ws, initial_state,
                       final_state, (bf16*)o, cu_seqlens, N, n_chunks, T, Hv, run);
  if (segmented) {
    hipLaunchKernelGGL(chunk_combine_kernel, dim3(N * Hv * (DV / CB_ROWS)), dim3(256), 0, s, run.local_final,
                       run.trans_final, s_start, final_state, Hv, run.G);
    hipLaunchKernelGGL((chunk_correct_kernel<bf16>), dim3(N * (run.G - 1) * Hv * run.Cs), dim3(256), 0, s, s_start,
                       run.trans_out, (bf16*)o, T, Hv, run.G, run.Cs);
  }
  return check_launch(fn);
}

// Scratch of zgdn_chunk_fwd_noalloc: the chunked path's workspace in a file-scope device array, one copy per
// device, allocated when the library's code object is loaded on that device and held until the process ends.
// Host code never passes the array's name to a kernel (that is a host-side stand-in, not a device address): it
// uses the address hipGetSymbolAddress returns for the current device, obtained once per device.
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)64 << 20;
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

constexpr int NOALLOC_MAX_DEVICES = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[NOALLOC_MAX_DEVICES] = {};

// The scratch's device address on the current device (looked up on the first call per device) into *out;
// returns ZGDN_OK, or the status recorded with the error.
int scratch_on_current_device(const char* fn, void** out) {
  *out = nullptr;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(ZGDN_EHIP, "%s: hipGetDevice: %s", fn, hipGetErrorString(e));
  if (dev < 0 || dev >= NOALLOC_MAX_DEVICES)
    return fail(ZGDN_EUNSUPPORTED, "%s: device %d (supported: 0 .. %d)", fn, dev, NOALLOC_MAX_DEVICES - 1);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return fail(ZGDN_EHIP, "%s: hipGetSymbolAddress(scratch) on device %d: %s", fn, dev,
                  e != hipSuccess ? hipGetErrorString(e) : "null address");
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return ZGDN_OK;
}
}  // namespace
}  // namespace zgdn

extern "C" int zgdn_chunk_fwd(const void* q, const void* k, const void* v, int qkv_dtype, const void* g,
                              const void* beta, int gb_dtype, const float* A_log, const float* dt_bias,
                              int qk_l2norm, const float* initial_state, float* final_state, void* o,
                              const int32_t* cu_seqlens, const int32_t* chunk_indices, int n_seqs, int n_chunks,
                              int B, int T, int Hk, int Hv, int K, int V, long q_ld, long k_ld, long v_ld,
                              long gb_ld, int beta_sigmoid, float scale, void* workspace, size_t workspace_bytes,
                              void* stream) {
  return zgdn::chunk_fwd_impl("zgdn_chunk_fwd", q, k, v, qkv_dtype, g, beta, gb_dtype, A_log, dt_bias, qk_l2norm,
                              initial_state, final_state, o, cu_seqlens, chunk_indices, n_seqs, n_chunks, B, T, Hk,
                              Hv, K, V, q_ld, k_ld, v_ld, gb_ld, beta_sigmoid, scale, workspace, workspace_bytes,
                              stream);
}

extern "C" size_t zgdn_chunk_noalloc_max_bytes(void) { return zgdn::NOALLOC_SCRATCH_BYTES; }

extern "C" int zgdn_chunk_fwd_noalloc(const void* q, const void* k, const void* v, int qkv_dtype, const void* g,
                                      const void* beta, int gb_dtype, const float* A_log, const float* dt_bias,
                                      int qk_l2norm, const float* initial_state, float* final_state, void* o,
                                      const int32_t* cu_seqlens, const int32_t* chunk_indices, int n_seqs,
                                      int n_chunks, int B, int T, int Hk, int Hv, int K, int V, long q_ld, long k_ld,
                                      long v_ld, long gb_ld, int beta_sigmoid, float scale, void* stream) {
  using namespace zgdn;
  const char* fn = "zgdn_chunk_fwd_noalloc";
  const int nc = cu_seqlens != nullptr ? n_chunks : (B > 0 && T >= 0 ? B * ((T + CH - 1) / CH) : 0);
  if (nc < 0 || Hv < 1) return fail(ZGDN_EINVAL, "%s: n_chunks=%d Hv=%d", fn, nc, Hv);
  const size_t need = zgdn_chunk_workspace_bytes(nc, Hv, K, V, qkv_dtype);  // 0: unsupported, refused below
  if (need > NOALLOC_SCRATCH_BYTES)
    return fail(ZGDN_EINVAL, "%s: %d chunks x %d heads need %zu bytes of workspace, above the %zu-byte scratch "
                "of this entry point (use zgdn_chunk_fwd with a caller workspace)", fn, nc, Hv, need,
                NOALLOC_SCRATCH_BYTES);
  void* ptr = nullptr;
  const int st = scratch_on_current_device(fn, &ptr);
  if (st != ZGDN_OK) return st;
  // the segmented state pass's extra space when it fits the scratch as well, else the plain pass
  size_t bytes = need;
  if (cu_seqlens == nullptr && B > 0 && T > 0 && qkv_dtype == ZGDN_BF16 && K == DK) {
    const size_t seg = zgdn_chunk_segment_workspace_size(B, T, Hv);
    if (seg > 0 && need + seg <= NOALLOC_SCRATCH_BYTES) bytes = need + seg;
  }
  return chunk_fwd_impl(fn, q, k, v, qkv_dtype, g, beta, gb_dtype, A_log, dt_bias, qk_l2norm, initial_state,
                        final_state, o, cu_seqlens, chunk_indices, n_seqs, n_chunks, B, T, Hk, Hv, K, V, q_ld,
                        k_ld, v_ld, gb_ld, beta_sigmoid, scale, ptr, bytes, stream);
}
