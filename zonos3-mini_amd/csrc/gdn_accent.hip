// Accent adapter shift of a projection: y_out = y_in + ((x . down^T) * mask) . up, per row, with the
// rounding points of the reference's bf16 torch ops (servers/sgl/src/zonos3_sgl/layers/accent.py:25-62:
// x @ down.T rounded, times mask rounded, @ up rounded, added to y rounded).
//
// Two launches. The down kernel (accent_down_lds_kernel, staged through LDS, for inputs of at most 1024 and
// adapters of rank up to 64; accent_down_bf16_kernel otherwise) forms tm = round(round(x . down^T) * mask)
// [rows, Kp] (Kp = K rounded up to 32, zero columns past K) into a small workspace; accent_up_kernel streams y: each workgroup forms
// y_out = y_in + round(tm . up) for 64-row x 128-column blocks (y_out may be y_in), reading up in place. Both
// run on bf16 MFMA (v_mfma_f32_16x16x32_bf16, fp32 accumulation) for bf16; fp32 runs plain fp32 arithmetic.
// Every row is computed on its own in a fixed order, so a row's result never depends on the other rows of
// the call (the batch invariance the reference gets by padding to fixed-row blocks).
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "gdn_common.h"

namespace zgdn {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int AC_ROWS = 64;   // rows per workgroup (16 per wave)
constexpr int AC_NB = 128;    // output columns per phase-2 workgroup
constexpr int AC_KMAX = 256;  // adapter columns (sum of the loaded adapters' ranks)

__device__ __forceinline__ int kpad(int K) { return (K + 31) / 32 * 32; }

__device__ __forceinline__ float rbf(float x) { return bf16_to_f32(f32_to_bf16(x)); }

__device__ __forceinline__ f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// 16 bytes at p, or zeros when !ok (p must then still be a valid address).
__device__ __forceinline__ bf16x8 load8(const uint16_t* p, bool ok) {
  const uint4 w = *reinterpret_cast<const uint4*>(p);
  return __builtin_bit_cast(bf16x8, ok ? w : make_uint4(0, 0, 0, 0));
}

// Loads in both kernels are issued by every lane from clamped, always-valid addresses: a load under a lane
// condition gets a wait for every outstanding load at its join, which would serialize the workgroup's round
// trips. Values read for rows past the batch or columns past the output are never stored; the only loads
// that must read as zero (the input tail when in is not a multiple of 32, up's rows past K) are selected
// after the load.
// tm[r][k] = round(round(sum_i x[r][i] down[k][i]) * mask[r][k]) for 16 rows per workgroup and every k < Kp.
// The input width is split over the workgroup's DW waves, each taking a contiguous run of 32-input steps
// (MFMA D tiles of 16 rows x 16 columns k: lane holds rows 4 (l / 16) + j, column l % 16) and issuing the
// loads of several steps at once, so that a workgroup waits about one memory round trip instead of one per
// step; the partial tiles are added in wave order through LDS, the same order for every row. (Staging down
// through LDS with contiguous loads, or 64 rows a workgroup sharing it, measured slower.)
// Waves per row block: 16 up to NT = 4, then 64 / NT (the partial tiles' LDS stays at 64 KiB).
template <int NT>
constexpr int down_waves() { return NT <= 4 ? 16 : 64 / NT; }
// input steps whose loads a wave issues at once (two for K <= 64: the 1024-input projection's 32 steps in one
// round trip of 16 waves)
template <int NT>
constexpr int down_steps() { return NT >= 8 ? 1 : 8 / NT; }

template <int NT, bool TAIL>  // TAIL: in is not a multiple of 32
__global__ __launch_bounds__(64 * down_waves<NT>()) void accent_down_bf16_kernel(
    const uint16_t* __restrict__ x, long x_ld, const uint16_t* __restrict__ down, const uint16_t* __restrict__ mask,
    long mask_ld, uint16_t* __restrict__ tm, int rows, int in, int K) {
  constexpr int DW = down_waves<NT>(), DSTEPS = down_steps<NT>();
  __shared__ f32x4 part[DW][NT][64];
  const int Kp = kpad(K);
  const int l = threadIdx.x & 63, wave = wave_id(), tid = threadIdx.x;
  const int r0 = blockIdx.x * 16;
  const int ra = min(r0 + (l & 15), rows - 1);
  const int steps = (in + 31) / 32, per = (steps + DW - 1) / DW;
  const int s0 = wave * per, s1 = min(steps, s0 + per);
  // the mask values of this thread's output elements (see the end), read with the block's first loads
  constexpr int FE = (16 * 16 * NT + 64 * DW - 1) / (64 * DW);  // output elements per thread, at most
  uint16_t mk[FE];
#pragma unroll
  for (int j = 0; j < FE; ++j) {
    const int e = tid + 64 * DW * j;
    mk[j] = mask[(size_t)min(r0 + e / Kp, rows - 1) * mask_ld + min(e % Kp, K - 1)];
  }
  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto batch = [&](int sb) {
    bf16x8 a[DSTEPS], b[DSTEPS][NT];
#pragma unroll
    for (int u = 0; u < DSTEPS; ++u) {
      // (a step past this wave's run re-reads its last step; its products are not added)
      const int i = 32 * min(sb + u, s1 - 1) + 8 * (l >> 4), ic = min(i, in - 8);
      a[u] = load8(x + (size_t)ra * x_ld + ic, !TAIL || i < in);
#pragma unroll
      for (int t = 0; t < NT; ++t) b[u][t] = load8(down + (size_t)min(16 * t + (l & 15), K - 1) * in + ic, true);
    }
    // every MFMA runs (so that no load sits under a condition); a step past the run keeps the old sums, and
    // tiles past Kp / 16 (NT = 8 with Kp = 96) are never read
#pragma unroll
    for (int u = 0; u < DSTEPS; ++u) {
      const bool live = sb + u < s1;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const f32x4 r = mfma_bf16(a[u], b[u][t], acc[t]);
        acc[t] = live ? r : acc[t];
      }
    }
  };
  // a run of at most DSTEPS steps (the 1024-input projection's) as straight-line code: in a loop the compiler
  // keeps the loads of one iteration from overlapping the earlier ones' (waits for reused registers)
  if (s1 - s0 <= DSTEPS) {
    if (s0 < s1) batch(s0);
  } else {
    for (int sb = s0; sb < s1; sb += DSTEPS) batch(sb);
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) part[wave][t][l] = acc[t];
  __syncthreads();
  // thread e finishes element (row e / Kp, column e % Kp) of the block: the DW partial tiles in wave order,
  // rounded, times the mask, rounded (columns past K: zero)
#pragma unroll
  for (int j = 0; j < FE; ++j) {
    const int e = tid + 64 * DW * j;
    const int rl = e / Kp, k = e % Kp, r = r0 + rl, t = k >> 4, L = 16 * (rl >> 2) + (k & 15);
    if (e >= 16 * Kp || r >= rows) break;
    float sum = part[0][t][L][rl & 3];
#pragma unroll
    for (int w = 1; w < DW; ++w) sum += part[w][t][L][rl & 3];
    tm[(size_t)r * Kp + k] = k < K ? f32_to_bf16(rbf(sum) * bf16_to_f32(mk[j])) : (uint16_t)0;
  }
}

// The staged form of the same product, for inputs of at most 1024 and Kp <= 64 (the projections' 1024 and 512
// inputs, adapters of rank up to 64): the block's 16 rows of x and down's Kp rows are read with coalesced
// 16-byte loads (a wave reads 1 KiB of one row) into an LDS copy, 16-byte chunk c of row r at c ^ (r % 16), and
// the MFMA fragments come from there. (Fragment loads straight from memory touch 16 rows 2 KiB apart per
// instruction: measured 15.5 bytes per cycle per CU against 50-56 for coalesced reads of the same data.) Each
// wave takes the same run of 32-input steps in the same MFMA order as accent_down_bf16_kernel and the partial
// tiles are added in wave order, so the sums are the same; chunks past the input width are stored as zeros.
constexpr int AC_LDS_CPR = 128;  // 16-byte chunks per staged row (in <= 1024)
template <int NT>
constexpr size_t down_lds_bytes() { return (size_t)(16 + 16 * NT) * AC_LDS_CPR * 16; }
template <int NT>
__global__ __launch_bounds__(1024) void accent_down_lds_kernel(const uint16_t* __restrict__ x, long x_ld,
                                                               const uint16_t* __restrict__ down,
                                                               const uint16_t* __restrict__ mask, long mask_ld,
                                                               uint16_t* __restrict__ tm, int rows, int in, int K) {
  constexpr int DW = 16, CPR = AC_LDS_CPR;
  extern __shared__ uint4 lds4[];  // x [16][CPR], down [16 NT][CPR]; then the partial tiles [DW][NT][64]
  const int Kp = kpad(K);
  const int l = threadIdx.x & 63, wave = wave_id(), tid = threadIdx.x;
  const int r0 = blockIdx.x * 16;
  const int cpr = in / 8, steps = (in + 31) / 32, per = (steps + DW - 1) / DW;
  const int s0 = wave * per, s1 = min(steps, s0 + per);
  constexpr int FE = (16 * 16 * NT + 64 * DW - 1) / (64 * DW);  // output elements per thread, at most
  uint16_t mk[FE];
#pragma unroll
  for (int j = 0; j < FE; ++j) {
    const int e = tid + 64 * DW * j;
    mk[j] = mask[(size_t)min(r0 + e / Kp, rows - 1) * mask_ld + min(e % Kp, K - 1)];
  }
  // every chunk of the staged rows: x's (rows past the batch re-read the last row, never stored) and down's
  // (rows past K re-read row K - 1: their columns of tm are written as zeros)
  constexpr int XJ = 16 * CPR / 1024, DJ = 16 * NT * CPR / 1024;
#pragma unroll
  for (int j = 0; j < XJ + DJ; ++j) {
    const int e = tid + 1024 * (j < XJ ? j : j - XJ), row = e / CPR, ch = e % CPR;
    const uint16_t* src = j < XJ ? x + (size_t)min(r0 + row, rows - 1) * x_ld : down + (size_t)min(row, K - 1) * in;
    const uint4 v = *reinterpret_cast<const uint4*>(src + 8 * min(ch, cpr - 1));
    // (a select of whole uint4 values is compiled into a scratch array indexed by the condition: per word)
    const uint32_t keep = ch < cpr ? ~0u : 0u;
    lds4[(j < XJ ? row : 16 + row) * CPR + (ch ^ (row & 15))] =
        make_uint4(v.x & keep, v.y & keep, v.z & keep, v.w & keep);
  }
  __syncthreads();
  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int m = l & 15, g = l >> 4;
  for (int st = s0; st < s1; ++st) {
    const int ch = 4 * st + g;
    const bf16x8 a = __builtin_bit_cast(bf16x8, lds4[m * CPR + (ch ^ m)]);
#pragma unroll
    for (int t = 0; t < NT; ++t)
      acc[t] = mfma_bf16(a, __builtin_bit_cast(bf16x8, lds4[(16 + 16 * t + m) * CPR + (ch ^ m)]), acc[t]);
  }
  __syncthreads();  // the partial tiles overwrite the staged rows
  f32x4* part = reinterpret_cast<f32x4*>(lds4);
#pragma unroll
  for (int t = 0; t < NT; ++t) part[(wave * NT + t) * 64 + l] = acc[t];
  __syncthreads();
  // thread e finishes element (row e / Kp, column e % Kp) of the block, as accent_down_bf16_kernel does
#pragma unroll
  for (int j = 0; j < FE; ++j) {
    const int e = tid + 64 * DW * j;
    const int rl = e / Kp, k = e % Kp, r = r0 + rl, t = k >> 4, L = 16 * (rl >> 2) + (k & 15);
    if (e >= 16 * Kp || r >= rows) break;
    float sum = part[t * 64 + L][rl & 3];
#pragma unroll
    for (int w = 1; w < DW; ++w) sum += part[(w * NT + t) * 64 + L][rl & 3];
    tm[(size_t)r * Kp + k] = k < K ? f32_to_bf16(rbf(sum) * bf16_to_f32(mk[j])) : (uint16_t)0;
  }
}

typedef short short4_t __attribute__((ext_vector_type(4)));
// Transposing LDS read (ds_read_b64_tr_b16): within each group of 16 lanes, lane s supplies the address of 4
// consecutive 16-bit elements (row k0 + s/4, columns c0 + 4 (s%4) .. +3 of a row-major matrix) and lane i
// receives column c0 + i of rows k0 .. k0 + 3.
__device__ __forceinline__ uint2 lds_tr(const uint16_t* p) {
  return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                       (__attribute__((address_space(3))) short4_t*)p));
}

// y_out[r][n] = round(y_in[r][n] + round(sum_k tm[r][k] up[k][n])) for AC_RB blocks of 64 rows x 128 columns.
// Every load of the workgroup is issued at its start -- its 128 columns of up (to LDS, row-major), the tm
// fragments and the y_in values of all its row blocks (16 bytes = 8 columns of one row per load, whole rows
// per instruction) -- so that it waits one memory round trip. Per block it forms the products on MFMA with
// the output columns as the M side (A = up^T, read from the row-major tile with transposing LDS reads) and the
// rows as the N side (B = tm rows), rounds them to bf16 through LDS in row order and adds them to its y
// values: every y access is 16 contiguous bytes. KS: 32-wide adapter steps held (Kp <= 32 KS).
constexpr int AC_RB = 1;  // 64-row blocks per phase-2 workgroup (2 measured 1 us slower, 4 slower still)
// Column blocks per row block: 128 columns each, a remainder of at most 8 columns folded into the last block
// (which keeps those 8 columns of up and of its products in the 8 pad columns of its LDS rows). A 2056-column
// projection then takes 16 blocks per row block instead of 17: 1024 workgroups for 4096 rows, one per slot at
// four workgroups a CU, where the 17th block of 8 columns made a second round of 64 workgroups.
__host__ __device__ inline int up_col_blocks(int out) {
  return out > AC_NB && out % AC_NB <= 8 ? out / AC_NB : (out + AC_NB - 1) / AC_NB;
}
template <bool HAS_Y, bool ALIGNED, int KS>
__global__ __launch_bounds__(256) void accent_up_bf16_kernel(const uint16_t* __restrict__ tm,
                                                             const uint16_t* __restrict__ up,
                                                             const uint16_t* y_in, long y_in_ld,
                                                             uint16_t* y_out, long y_out_ld, int rows,
                                                             int out, int K) {  // y_out may equal y_in
  constexpr int NB = AC_NB, SP = NB + 8;  // (row pitch of both LDS tiles: 272 bytes)
  extern __shared__ uint16_t lds[];        // up's tile [Kp][SP] (rows k, columns n0 ..), the products [AC_ROWS][SP]
  const int Kp = kpad(K);
  uint16_t* ut = lds;
  uint16_t* sh = lds + Kp * SP;
  // Workgroup ids go round-robin over the 8 XCDs: all column blocks of one row block take ids of one residue
  // mod 8, so they run on one XCD and share its L2 copy of the 128-byte lines their rows straddle (the
  // projection's rows are rarely line-aligned: 2056 bf16 = 4112 bytes).
  const int n_nb = up_col_blocks(out), n_rb = (rows + AC_ROWS * AC_RB - 1) / (AC_ROWS * AC_RB);
  const int xcd = blockIdx.x % 8, slot = blockIdx.x / 8;
  const int rblk = (slot / n_nb) * 8 + xcd, nblk = slot % n_nb;
  if (rblk >= n_rb) return;
  const int n0 = nblk * NB, rbase = rblk * (AC_ROWS * AC_RB);
  const bool wide = nblk == n_nb - 1 && n0 + NB < out;  // the last block, with folded columns n0 + NB .. +7
  const int tid = threadIdx.x, l = tid & 63, wave = wave_id();
  constexpr int G = NB / 8;               // 16-byte groups per row of y
  constexpr int PER = AC_ROWS * G / 256;  // y groups per thread and block
  constexpr int NT = NB / 16;
  // up rows k < Kp, columns n0 .. n0 + NB - 1 (for LDS: zeros past K, where tm is zero too, keep non-finite
  // values of up's last row out), loaded first so that their stores to LDS wait for these loads only
  constexpr int UPER = 32 * KS * G / 256;
  uint4 uw[UPER];
#pragma unroll
  for (int it = 0; it < UPER; ++it) {
    const int e = tid + 256 * it, k = e / G, c8 = 8 * (e % G);
    uw[it] = *reinterpret_cast<const uint4*>(up + (size_t)min(k, K - 1) * out + min(n0 + c8, out - 8));
  }
  static_assert(AC_RB == 1, "the folded columns are handled for one row block a workgroup");
  // the folded block's 8 extra columns of up (row tid), read by every workgroup from a clamped address so that
  // no load sits under a condition (the others never store it)
  const uint4 ux = *reinterpret_cast<const uint4*>(up + (size_t)min(tid, K - 1) * out + min(n0 + NB, out - 8));
  // then the tm fragments of every block (wave w: rows 16 w .. +15 of each block, the MFMA N side) and, last,
  // y_in of every block, so that the products' MFMA waits for the fragments only and the y loads stay in flight
  // through it. (Staging tm through LDS with coalesced loads, as the down kernel does with its operands,
  // measured slower here: 16 KiB a workgroup, against the extra LDS pass and barrier.)
  uint4 yw[AC_RB][PER];
  bf16x8 tb[AC_RB][KS];
#pragma unroll
  for (int b = 0; b < AC_RB; ++b) {
    const int r0 = rbase + AC_ROWS * b;
    const int rb = min(r0 + 16 * wave + (l & 15), rows - 1);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) tb[b][ks] = load8(tm + (size_t)rb * Kp + min(32 * ks + 8 * (l >> 4), Kp - 8), true);
  }
  auto load_y = [&](int r, int n) {
    if constexpr (!HAS_Y) return make_uint4(0, 0, 0, 0);
    const uint16_t* yp = y_in + (size_t)min(r, rows - 1) * y_in_ld + min(n, out - 8);
    if constexpr (ALIGNED) return *reinterpret_cast<const uint4*>(yp);
    uint32_t u[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) u[j] = (uint32_t)yp[2 * j] | ((uint32_t)yp[2 * j + 1] << 16);
    return make_uint4(u[0], u[1], u[2], u[3]);
  };
#pragma unroll
  for (int b = 0; b < AC_RB; ++b) {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int e = tid + 256 * p;
      yw[b][p] = load_y(rbase + AC_ROWS * b + e / G, n0 + 8 * (e % G));
    }
  }
  const uint4 yx = load_y(rbase + (tid & (AC_ROWS - 1)), n0 + NB);  // the folded columns' y_in (row tid)
#pragma unroll
  for (int it = 0; it < UPER; ++it) {
    const int e = tid + 256 * it, k = e / G, c8 = 8 * (e % G);
    if (k < Kp) *reinterpret_cast<uint4*>(&ut[k * SP + c8]) = k < K ? uw[it] : make_uint4(0, 0, 0, 0);
  }
  if (wide && tid < Kp) *reinterpret_cast<uint4*>(&ut[tid * SP + NB]) = tid < K ? ux : make_uint4(0, 0, 0, 0);
  __syncthreads();

#pragma unroll
  for (int b = 0; b < AC_RB; ++b) {
    const int r0 = rbase + AC_ROWS * b;
    if (r0 >= rows) break;
    f32x4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int sl = l & 15;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (32 * ks >= Kp) break;
      // A fragment: column n0 + 16 t + l % 16 of up, k = 32 ks + 8 (l / 16) .. +7 (two transposing reads)
      const int k0 = 32 * ks + 8 * (l >> 4) + (sl >> 2);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint2 a0 = lds_tr(&ut[k0 * SP + 16 * t + 4 * (sl & 3)]);
        const uint2 a1 = lds_tr(&ut[(k0 + 4) * SP + 16 * t + 4 * (sl & 3)]);
        acc[t] = mfma_bf16(__builtin_bit_cast(bf16x8, make_uint4(a0.x, a0.y, a1.x, a1.y)), tb[b][ks], acc[t]);
      }
    }
    // D: lane holds columns 16 t + 4 (l / 16) + j of row 16 w + l % 16: rounded products to LDS
    const int rr = 16 * wave + (l & 15);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int c = 16 * t + 4 * (l >> 4);
      *reinterpret_cast<uint2*>(&sh[rr * SP + c]) =
          make_uint2(pack_bf16x2(acc[t][0], acc[t][1]), pack_bf16x2(acc[t][2], acc[t][3]));
    }
    // the folded columns as a ninth column tile whose last 8 columns repeat its first 8 (lanes with column
    // offsets 8 .. 15 read 0 .. 7: every read stays inside the 8 pad columns of the row), those never stored
    if (wide) {  // (after the other tiles are stored, in their registers)
      f32x4 accx = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if (32 * ks >= Kp) break;
        const int k0 = 32 * ks + 8 * (l >> 4) + (sl >> 2);
        const uint2 a0 = lds_tr(&ut[k0 * SP + NB + 4 * (sl & 1)]);
        const uint2 a1 = lds_tr(&ut[(k0 + 4) * SP + NB + 4 * (sl & 1)]);
        accx = mfma_bf16(__builtin_bit_cast(bf16x8, make_uint4(a0.x, a0.y, a1.x, a1.y)), tb[b][ks], accx);
      }
      if ((l >> 4) < 2)
        *reinterpret_cast<uint2*>(&sh[rr * SP + NB + 4 * (l >> 4)]) =
            make_uint2(pack_bf16x2(accx[0], accx[1]), pack_bf16x2(accx[2], accx[3]));
    }
    __syncthreads();
    // y_out = y_in + products for 8 columns (local row rl, local column cl) of the block
    auto finish = [&](int rl, int cl, const uint4& yv) {
      const uint4 sw = *reinterpret_cast<const uint4*>(&sh[rl * SP + cl]);
      const uint32_t su[4] = {sw.x, sw.y, sw.z, sw.w}, yu[4] = {yv.x, yv.y, yv.z, yv.w};
      uint32_t ou[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float s_lo = __uint_as_float(su[j] << 16), s_hi = __uint_as_float(su[j] & 0xffff0000u);
        const float y_lo = __uint_as_float(yu[j] << 16), y_hi = __uint_as_float(yu[j] & 0xffff0000u);
        ou[j] = HAS_Y ? pack_bf16x2(y_lo + s_lo, y_hi + s_hi) : su[j];
      }
      uint16_t* op = y_out + (size_t)(r0 + rl) * y_out_ld + n0 + cl;
      if constexpr (ALIGNED) {
        *reinterpret_cast<uint4*>(op) = make_uint4(ou[0], ou[1], ou[2], ou[3]);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          op[2 * j] = (uint16_t)(ou[j] & 0xffffu);
          op[2 * j + 1] = (uint16_t)(ou[j] >> 16);
        }
      }
    };
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int e = tid + 256 * p, rl = e / G, cl = 8 * (e % G);
      if (r0 + rl >= rows || n0 + cl >= out) continue;
      finish(rl, cl, yw[b][p]);
    }
    if (wide && tid < AC_ROWS && r0 + tid < rows) finish(tid, NB, yx);
    if (b + 1 < AC_RB) __syncthreads();  // the products' LDS is rewritten by the next block
  }
}

// fp32: one thread per (row, adapter column) / (row, output column), fp32 throughout.
__global__ __launch_bounds__(256) void accent_down_f32_kernel(const float* __restrict__ x, long x_ld,
                                                              const float* __restrict__ down,
                                                              const float* __restrict__ mask, long mask_ld,
                                                              float* __restrict__ tm, int rows, int in, int K) {
  const int Kp = kpad(K);
  const long e = (long)blockIdx.x * 256 + threadIdx.x;
  if (e >= (long)rows * Kp) return;
  const int r = (int)(e / Kp), k = (int)(e % Kp);
  float acc = 0.f;
  if (k < K) {
    for (int i = 0; i < in; ++i) acc = fmaf(x[(size_t)r * x_ld + i], down[(size_t)k * in + i], acc);
    acc *= mask[(size_t)r * mask_ld + k];
  }
  tm[(size_t)r * Kp + k] = acc;
}

__global__ __launch_bounds__(256) void accent_up_f32_kernel(const float* __restrict__ tm, const float* __restrict__ up,
                                                            const float* y_in, long y_in_ld, float* y_out,
                                                            long y_out_ld, int rows, int out, int K) {
  const int Kp = kpad(K);
  const long e = (long)blockIdx.x * 256 + threadIdx.x;
  if (e >= (long)rows * out) return;
  const int r = (int)(e / out), n = (int)(e % out);
  float acc = 0.f;
  for (int k = 0; k < K; ++k) acc = fmaf(tm[(size_t)r * Kp + k], up[(size_t)k * out + n], acc);
  y_out[(size_t)r * y_out_ld + n] = (y_in != nullptr ? y_in[(size_t)r * y_in_ld + n] : 0.f) + acc;
}

// The staged down kernel's dynamic LDS (96 or 160 KiB) is above the default 64 KiB: raised once per device (the
// first call on it); false when the device refuses, and the caller then takes the unstaged kernel.
constexpr int AC_MAX_DEVICES = 64;
template <int NT>
bool down_lds_ready() {
  static std::atomic<signed char> state[AC_MAX_DEVICES];  // 0 unknown, 1 ready, -1 refused
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= AC_MAX_DEVICES) return false;
  const signed char st = state[dev].load(std::memory_order_acquire);
  if (st != 0) return st > 0;
  const bool ok = hipFuncSetAttribute((const void*)accent_down_lds_kernel<NT>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      (int)down_lds_bytes<NT>()) == hipSuccess;
  if (!ok) (void)hipGetLastError();  // (clear the refused call's error for the launches that follow)
  state[dev].store(ok ? 1 : -1, std::memory_order_release);
  return ok;
}

}  // namespace
}  // namespace zgdn

extern "C" size_t zgdn_accent_workspace_size(int rows, int out, int K, int dtype) {
  if (rows <= 0 || out <= 0 || K <= 0) return 0;
  const size_t Kp = (size_t)((K + 31) / 32 * 32);
  // tm [rows, Kp]
  return (size_t)rows * Kp * (dtype == ZGDN_F32 ? 4 : 2);
}

extern "C" int zgdn_accent_shift(const void* x, long x_ld, const void* down, const void* up, const void* mask,
                                 long mask_ld, const void* y_in, long y_in_ld, void* y_out, long y_out_ld, int rows,
                                 int in, int out, int K, int dtype, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  using namespace zgdn;
  const char* fn = "zgdn_accent_shift";
  if (!x || !down || !up || !mask || !y_out || !workspace) return fail(ZGDN_EINVAL, "%s: null pointer", fn);
  if (dtype != ZGDN_F32 && dtype != ZGDN_BF16) return fail(ZGDN_EINVAL, "%s: dtype code %d", fn, dtype);
  if (rows < 0 || in < 1 || out < 1 || K < 1 || K > AC_KMAX)
    return fail(ZGDN_EUNSUPPORTED, "%s: rows=%d in=%d out=%d K=%d (K <= %d)", fn, rows, in, out, K, AC_KMAX);
  if (x_ld < in || mask_ld < K || y_out_ld < out || (y_in != nullptr && y_in_ld < out))
    return fail(ZGDN_EINVAL, "%s: row strides x=%ld mask=%ld y_in=%ld y_out=%ld below the row widths", fn, x_ld,
                mask_ld, y_in_ld, y_out_ld);
  const bool bf = dtype == ZGDN_BF16;
  if (bf && (in % 8 || out % 8 || x_ld % 8 || ((uintptr_t)x | (uintptr_t)down | (uintptr_t)up) % 16))
    return fail(ZGDN_EINVAL, "%s: bf16 needs in, out and the x row stride multiples of 8 and 16-byte aligned x, "
                "down, up (in=%d out=%d x_ld=%ld)", fn, in, out, x_ld);
  if (bf && (uintptr_t)workspace % 16) return fail(ZGDN_EINVAL, "%s: workspace not 16-byte aligned", fn);
  if (workspace_bytes < zgdn_accent_workspace_size(rows, out, K, dtype))
    return fail(ZGDN_EINVAL, "%s: workspace of %zu bytes, need %zu", fn, workspace_bytes,
                zgdn_accent_workspace_size(rows, out, K, dtype));
  if (rows == 0) return check_launch(fn);
  hipStream_t s = (hipStream_t)stream;
  const int Kp = (K + 31) / 32 * 32;
  if (bf) {
    const dim3 g1((rows + 15) / 16);  // row blocks of 16
    auto d = (const uint16_t*)down;
    auto m = (const uint16_t*)mask;
    auto tm = (uint16_t*)workspace;
    auto go1 = [&](auto nt) {
      constexpr int NT = decltype(nt)::value;  // MFMA column tiles per wave, Kp / 16 rounded up to a power of 2
      auto k1 = in % 32 ? accent_down_bf16_kernel<NT, true> : accent_down_bf16_kernel<NT, false>;
      hipLaunchKernelGGL(k1, g1, dim3(64 * down_waves<NT>()), 0, s, (const uint16_t*)x, x_ld, d, m, mask_ld, tm, rows,
                         in, K);
    };
    auto go_lds = [&](auto nt) -> bool {
      constexpr int NT = decltype(nt)::value;
      if (!down_lds_ready<NT>()) return false;
      hipLaunchKernelGGL((accent_down_lds_kernel<NT>), g1, dim3(1024), down_lds_bytes<NT>(), s, (const uint16_t*)x,
                         x_ld, d, m, mask_ld, tm, rows, in, K);
      return true;
    };
    // the staged kernel where its LDS copy holds the rows (in <= 1024, Kp <= 64), else the unstaged one
    const bool staged = in <= 8 * AC_LDS_CPR && Kp <= 64 &&
                        (Kp <= 32 ? go_lds(std::integral_constant<int, 2>{}) : go_lds(std::integral_constant<int, 4>{}));
    if (!staged) {
      if (Kp <= 32) go1(std::integral_constant<int, 2>{});
      else if (Kp <= 64) go1(std::integral_constant<int, 4>{});
      else if (Kp <= 128) go1(std::integral_constant<int, 8>{});
      else go1(std::integral_constant<int, 16>{});
    }
    const bool aligned = (((uintptr_t)y_out | (uintptr_t)(y_in ? y_in : y_out)) % 16 == 0) && y_out_ld % 8 == 0 &&
                         (y_in == nullptr || y_in_ld % 8 == 0);
    const int n_nb = up_col_blocks(out), n_rb = (rows + AC_ROWS * AC_RB - 1) / (AC_ROWS * AC_RB);
    const dim3 g2(8 * n_nb * ((n_rb + 7) / 8));  // XCD-grouped ids (see the kernel)
    const size_t lds = ((size_t)Kp + AC_ROWS) * (AC_NB + 8) * 2;  // <= 87,040 bytes
    auto pick = [&](auto ks) -> void (*)(const uint16_t*, const uint16_t*, const uint16_t*, long, uint16_t*, long,
                                         int, int, int) {
      constexpr int KS = decltype(ks)::value;
      return y_in != nullptr
                 ? (aligned ? accent_up_bf16_kernel<true, true, KS> : accent_up_bf16_kernel<true, false, KS>)
                 : (aligned ? accent_up_bf16_kernel<false, true, KS> : accent_up_bf16_kernel<false, false, KS>);
    };
    auto up2 = Kp <= 64 ? pick(std::integral_constant<int, 2>{}) : pick(std::integral_constant<int, 8>{});
    if (lds > 65536 &&
        hipFuncSetAttribute((const void*)up2, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return fail(ZGDN_EHIP, "%s: %zu bytes of LDS for K=%d not available", fn, lds, K);
    hipLaunchKernelGGL(up2, g2, dim3(256), lds, s, tm, (const uint16_t*)up, (const uint16_t*)y_in, y_in_ld,
                       (uint16_t*)y_out, y_out_ld, rows, out, K);
  } else {
    auto tm = (float*)workspace;
    const long n1 = (long)rows * Kp, n2 = (long)rows * out;
    hipLaunchKernelGGL(accent_down_f32_kernel, dim3((unsigned)((n1 + 255) / 256)), dim3(256), 0, s, (const float*)x,
                       x_ld, (const float*)down, (const float*)mask, mask_ld, tm, rows, in, K);
    hipLaunchKernelGGL(accent_up_f32_kernel, dim3((unsigned)((n2 + 255) / 256)), dim3(256), 0, s, tm,
                       (const float*)up, (const float*)y_in, y_in_ld, (float*)y_out, y_out_ld, rows, out, K);
  }
  return check_launch(fn);
}
