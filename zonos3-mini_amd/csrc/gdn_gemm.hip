// The GDN layer's projections on bf16 MFMA: Y = X W^T with X [M, K] (the tokens' rows), W [N, K] (the weight as
// stored, torch's F.linear layout) and Y [M, N], bf16 in and out, fp32 accumulation (lm.py:561 in_proj, lm.py:602
// wo; servers/sgl/src/zonos3_sgl/models/gdn.py:399, 447), and in_proj with the depthwise causal conv + SiLU of
// its q|k|v columns applied in the epilogue (lm.py:561-568), so that the projection's raw q|k|v never goes to
// memory and the conv needs no pass of its own.
//
// Both operands are K-contiguous, so an MFMA fragment (v_mfma_f32_16x16x32_bf16: lane 16 g + m holds 8
// consecutive k of row m of A, or of column m of B, i.e. of row m of W) is one 16-byte read of a row. Workgroups
// of 8 waves own BM x 128 output tiles (the launches use BM = 128: waves 2 x 4 of 64 x 32; the configuration also
// describes BM = 256: waves 4 x 2 of 64 x 64) and
// walk K in blocks of 64 staged through LDS (128-byte rows, 16-byte chunk c of row r at c ^ ((r / 2) % 8), which
// keeps the 16-row fragment reads free of bank conflicts), filled by direct-to-LDS loads (buffer_load_dwordx4 ...
// lds): block kb computes while the next blocks land (three stages for 256-row tiles, one workgroup per CU; two
// for 128-row tiles, two workgroups per CU). Tiles are grouped so that
// the workgroups of one XCD (workgroups go round-robin over the 8 XCDs) share a 4 x 8 block of tiles and read
// their operands once into that XCD's L2. Columns past the last multiple of 128 (in_proj's a | b: 2056 = 16 x 128
// + 8) are taken by a strip kernel.
//
// Conv tiles (columns below C, the q|k|v channels): the conv of row t reads the raw projection of rows t - 3 ..
// t, so a tile past the first also computes the 16 rows above it (one more 16 x 16 MFMA tile per wave, with a B
// fragment the wave holds anyway: +1/16 of the tile's MFMAs), rounded to bf16 as the projection itself; the first
// tile takes rows -3 .. -1 from the conv history. The epilogue stages the tile's bf16 projection (halo rows
// first) in LDS and each thread runs the conv down a 2-channel strip of BM / 8 rows with the arithmetic of the
// conv kernel of gdn_rowops.hip (taps oldest first, fma chain in fp32, rounded to bf16, SiLU, rounded again).
// The tile holding the last rows writes the new history (the last 3 raw rows, oldest first).
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "gdn_common.h"

namespace zgdn {
namespace {

typedef __bf16 gbf16x8 __attribute__((ext_vector_type(8)));
typedef float gf32x4 __attribute__((ext_vector_type(4)));

constexpr int GK = 64;         // K block (two MFMA k-steps)
constexpr int GBN = 128;       // tile columns
constexpr int GTHREADS = 512;  // 8 waves
constexpr int HALO = 16;       // rows above a conv tile computed again
constexpr int CW = 4;          // conv width (the model's GDN_KERNEL)

__device__ __forceinline__ gf32x4 gmfma(gbf16x8 a, gbf16x8 b, gf32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Byte offset of 16-byte chunk c (0..7) of row r in a block of 128-byte rows.
__device__ __forceinline__ int gsw(int r, int c) { return r * 128 + ((c ^ ((r >> 1) & 7)) << 4); }

template <int BM>
struct GemmCfg {
  static constexpr int WGM = BM == 256 ? 4 : 2;  // waves along M
  static constexpr int WGN = 8 / WGM;            // waves along N
  static constexpr int TM = BM / WGM / 16;       // 16-row tiles per wave
  static constexpr int TN = GBN / WGN / 16;      // 16-column tiles per wave
  static constexpr int B_PIECES = GBN * 128 / 1024;
  // A stage: the A rows (halo rows first), W's tile rows, and with R 16 rows of W past the full column tiles
  // (the remainder strip: rows beyond N read zero); in 1 KiB pieces of 8 rows
  template <bool H, bool R>
  struct St {
    static constexpr int HB = H ? HALO : 0;
    static constexpr int A_PIECES = (HB + BM) / 8;
    static constexpr int R_PIECES = R ? 2 : 0;
    static constexpr int PIECES = A_PIECES + B_PIECES + R_PIECES;
    static constexpr int BYTES = PIECES * 1024;
    static constexpr int MAXP = (PIECES + 7) / 8;  // pieces per wave (at most)
  };
  // LDS stages: three for 256-row tiles (one workgroup per CU), two for 128-row tiles (two workgroups per CU,
  // so that one's epilogue runs beside the other's MFMAs)
  static constexpr int STAGES = BM == 256 ? 3 : 2;
  static constexpr int WG_PER_CU = BM == 256 ? 1 : 2;
  static constexpr int LDS = STAGES * St<true, true>::BYTES;
};

// A stage's pieces: piece p (1 KiB of LDS at stage + 1024 p) goes to wave p % 8; pieces below A_PIECES hold rows
// 8 p .. of the tile's A rows (from row m0 - HB of X), the others rows of W's tile. One wave instruction fills a
// piece, lane i at +16 i, so each lane fetches the 16-byte chunk that the swizzled layout puts at its position.
// Buffer resources over the tile's rows (rows past M or N read zero; their products are never stored); the K
// block goes in the scalar offset.
template <int BM, bool H, bool R>
struct TileSrc {
  using S = typename GemmCfg<BM>::template St<H, R>;
  // per slot: the base address and byte count of the resource its piece reads through (selected as integers:
  // a choice among three resources is lowered through a private array in scratch), and this lane's offset
  uint64_t base[S::MAXP];
  uint32_t bytes[S::MAXP];
  uint32_t off[S::MAXP];
};

template <int BM, bool H, bool R>
__device__ __forceinline__ TileSrc<BM, H, R> tile_src(const uint16_t* X, long x_ld, const uint16_t* W, long K, int m0,
                                                      int n0, int M, int N, int n_rem0) {
  using S = typename GemmCfg<BM>::template St<H, R>;
  TileSrc<BM, H, R> t;
  const int ma = m0 - S::HB;  // first A row (>= 0: the halo form is not used for the first tile)
  // (byte counts through readfirstlane: the compiler forms the clamps with vector instructions, and a resource
  // built from a vector register turns every load into a loop over the lanes' values)
  const uint32_t xb = (uint32_t)__builtin_amdgcn_readfirstlane(
      (int)((uint32_t)max(min(S::HB + BM, M - ma), 0) * (uint32_t)x_ld * 2u));
  const uint32_t wb =
      (uint32_t)__builtin_amdgcn_readfirstlane((int)((uint32_t)max(min(GBN, N - n0), 0) * (uint32_t)K * 2u));
  const uint64_t xa = (uint64_t)(X + (size_t)ma * x_ld), wa = (uint64_t)(W + (size_t)n0 * K);
  uint64_t ra = wa;
  uint32_t rb = 0;
  if constexpr (R) {
    rb = (uint32_t)__builtin_amdgcn_readfirstlane((int)((uint32_t)max(min(16, N - n_rem0), 0) * (uint32_t)K * 2u));
    ra = (uint64_t)(W + (size_t)n_rem0 * K);
  }
  const int wave = wave_id(), i = threadIdx.x & 63;
#pragma unroll
  for (int s = 0; s < S::MAXP; ++s) {
    const int p = wave + 8 * s;
    const bool is_a = p < S::A_PIECES, is_b = !is_a && p < S::A_PIECES + GemmCfg<BM>::B_PIECES;
    const int q = is_a ? p : (is_b ? p - S::A_PIECES : p - S::A_PIECES - GemmCfg<BM>::B_PIECES);
    const int r = 8 * q + (i >> 3), c = (i & 7) ^ ((r >> 1) & 7);
    t.off[s] = (uint32_t)r * (uint32_t)(is_a ? x_ld : K) * 2u + 16u * c;
    t.base[s] = is_a ? xa : (is_b ? wa : ra);
    t.bytes[s] = is_a ? xb : (is_b ? wb : rb);
  }
  return t;
}

// Issues this wave's loads of K block kb into `stage`.
template <int BM, bool H, bool R>
__device__ __forceinline__ void gload_lds(const TileSrc<BM, H, R>& t, uint8_t* stage, int kb, int wave) {
  using S = typename GemmCfg<BM>::template St<H, R>;
  typedef __attribute__((address_space(3))) void* lptr;
  const uint32_t k = (uint32_t)kb * GK * 2u;
#pragma unroll
  for (int s = 0; s < S::MAXP; ++s) {
    const int p = wave + 8 * s;
    if (p < S::PIECES)  // (wave-uniform)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(raw_rsrc((const void*)t.base[s], t.bytes[s]), (lptr)(stage + 1024 * p),
                                               16, t.off[s], k, 0, 0);
  }
}

// Waits until at most n of this wave's loads are outstanding (n: its pieces of one block, 4 .. 7).
__device__ __forceinline__ void wait_pieces(int n) {
  if (n >= 7)
    asm volatile("s_waitcnt vmcnt(7)" ::: "memory");
  else if (n == 6)
    asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
  else if (n == 5)
    asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
  else
    asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
}

__device__ __forceinline__ void lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int BM>
using Acc = gf32x4[GemmCfg<BM>::TM][GemmCfg<BM>::TN];

// The K loop of one tile: acc gets this wave's TM x TN tiles; with H, hacc the halo tile (rows -16 .. -1, the
// wave's column tile wm); with R, the wave holding tile rows 16 r_row .. (r_row = the tile's column index)
// forms racc, those rows of the remainder strip. Ends with
// every load done and a barrier (the LDS is then free for the epilogue).
template <int BM, bool H, bool R>
__device__ __forceinline__ void k_loop(const uint16_t* X, long x_ld, const uint16_t* W, int M, int N, int K, int m0,
                                       int n0, int n_rem0, uint8_t* lds, Acc<BM>& acc, gf32x4& hacc, gf32x4& racc,
                                       int wr0, int wc0, int wm, int wave, int r_row) {
  using C = GemmCfg<BM>;
  using S = typename C::template St<H, R>;
  const TileSrc<BM, H, R> src = tile_src<BM, H, R>(X, x_ld, W, K, m0, n0, M, N, n_rem0);
  const bool r_wave = R && wave == r_row / C::TM;  // (wave-uniform)
  const int nk = K / GK;
  const int mine = (S::PIECES - wave + 7) / 8;  // this wave's pieces per block
  const int l = threadIdx.x & 63, m = l & 15, g = l >> 4;
  constexpr int NS = C::STAGES;
#pragma unroll
  for (int q = 0; q < NS - 1; ++q) gload_lds<BM, H, R>(src, lds + q * S::BYTES, min(q, nk - 1), wave);
  // Block kb computes from stage kb % NS. A wave waits for its own loads of block kb (those of the blocks after
  // it may stay outstanding), the barrier for everyone's and for every wave to be done with the stage the next
  // loads overwrite. Past the last block the last one is loaded again (into a stage nothing reads), so that the
  // wait count stays the same.
  int st = 0;
  for (int kb = 0; kb < nk; ++kb) {
    if constexpr (NS == 3)
      wait_pieces(mine);
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    const int stn = st == 0 ? NS - 1 : st - 1;  // stage of block kb + NS - 1 (= that of block kb - 1)
    gload_lds<BM, H, R>(src, lds + stn * S::BYTES, min(kb + NS - 1, nk - 1), wave);
    const uint8_t* a_st = lds + st * S::BYTES;
    const uint8_t* b_st = a_st + S::A_PIECES * 1024;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      gbf16x8 a[C::TM], b[C::TN];
#pragma unroll
      for (int i = 0; i < C::TM; ++i)
        a[i] = *reinterpret_cast<const gbf16x8*>(a_st + gsw(S::HB + wr0 + 16 * i + m, 4 * s + g));
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
        b[j] = *reinterpret_cast<const gbf16x8*>(b_st + gsw(wc0 + 16 * j + m, 4 * s + g));
#pragma unroll
      for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int j = 0; j < C::TN; ++j) acc[i][j] = gmfma(a[i], b[j], acc[i][j]);
      if constexpr (H) {
        const gbf16x8 ah = *reinterpret_cast<const gbf16x8*>(a_st + gsw(m, 4 * s + g));
        gbf16x8 bh = b[0];
#pragma unroll
        for (int j = 1; j < C::TN; ++j)
          if (j == wm) bh = b[j];  // (wave-uniform selection of the wave's column tile wm)
        hacc = gmfma(ah, bh, hacc);
      }
      if constexpr (R) {
        if (r_wave) {  // (its A fragment read again: selecting a[r_i] by a run-time index spills the array)
          const gbf16x8 br = *reinterpret_cast<const gbf16x8*>(b_st + C::B_PIECES * 1024 + gsw(m, 4 * s + g));
          const gbf16x8 ar = *reinterpret_cast<const gbf16x8*>(a_st + gsw(S::HB + 16 * r_row + m, 4 * s + g));
          racc = gmfma(ar, br, racc);
        }
      }
    }
    st = st == NS - 1 ? 0 : st + 1;
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
}

// This wave's D tiles rounded to bf16 into the LDS tile `out` (rows of 128 bf16, starting at row `row0`).
template <int BM>
__device__ __forceinline__ void stage_out(uint16_t* out, int row0, const Acc<BM>& acc, int wr0, int wc0) {
  using C = GemmCfg<BM>;
  const int l = threadIdx.x & 63, m = l & 15, g = l >> 4;
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        out[(row0 + wr0 + 16 * i + 4 * g + e) * GBN + wc0 + 16 * j + m] = f32_to_bf16(acc[i][j][e]);
}

// Full BM x 128 tiles (K a multiple of 64). CONV: the tiles of columns below C get the conv epilogue. R: the
// columns past the full tiles (at most 16) are formed by the tiles themselves, tile (tm, tn) their rows
// 16 tn .. 16 tn + 15 of row block tm (the host takes R when the column tiles cover the row block so).
// (X and W are not __restrict__: as restrict-qualified read-only data their loads could be moved past the LDS
// barriers.)
template <int BM, bool CONV, bool R>
__global__ __launch_bounds__(GTHREADS, GemmCfg<BM>::WG_PER_CU) void gemm_kernel(const uint16_t* X, long x_ld, const uint16_t* W,
                                                           uint16_t* __restrict__ Y, long y_ld, int M, int N, int K,
                                                           int tiles_m, int tiles_n, const uint16_t* __restrict__ conv_w,
                                                           int C, const uint16_t* __restrict__ hist_in,
                                                           uint16_t* __restrict__ hist_out) {
  using G = GemmCfg<BM>;
  extern __shared__ uint4 glds[];
  uint8_t* lds = reinterpret_cast<uint8_t*>(glds);
  // tile order: the 8 XCDs take workgroups round-robin; XCD x gets a 4 x 8 block of tiles when the grid is 256
  // tiles of such blocks, else a run of row blocks
  const int id = blockIdx.x, n_full = tiles_m * tiles_n;
  const int xcd = id & 7, slot = id >> 3, per_xcd = n_full / 8;
  int tm, tn;
  if (per_xcd == 32 && tiles_m % 4 == 0 && tiles_n % 8 == 0) {
    const int bands_n = tiles_n / 8;
    tm = (xcd / bands_n) * 4 + slot / 8;
    tn = (xcd % bands_n) * 8 + slot % 8;
  } else if (per_xcd * 8 == n_full && per_xcd % tiles_n == 0) {
    const int t = xcd * per_xcd + slot;
    tm = t / tiles_n;
    tn = t % tiles_n;
  } else {
    tm = id / tiles_n;
    tn = id % tiles_n;
  }
  // (wave-uniform values kept in scalar registers: the buffer resources built from them must be scalar)
  const int m0 = __builtin_amdgcn_readfirstlane(tm * BM), n0 = __builtin_amdgcn_readfirstlane(tn * GBN);
  const int wave = wave_id(), wm = wave % G::WGM, wn = wave / G::WGM;
  const int wr0 = wm * G::TM * 16, wc0 = wn * G::TN * 16;
  const int l = threadIdx.x & 63, m = l & 15, g = l >> 4;

  Acc<BM> acc;
#pragma unroll
  for (int i = 0; i < G::TM; ++i)
#pragma unroll
    for (int j = 0; j < G::TN; ++j) acc[i][j] = gf32x4{0.f, 0.f, 0.f, 0.f};
  gf32x4 hacc = {0.f, 0.f, 0.f, 0.f}, racc = {0.f, 0.f, 0.f, 0.f};
  const bool conv = CONV && n0 < C;
  const int n_rem0 = tiles_n * GBN;
  const bool rem = R && 16 * tn < BM;  // this tile forms rows 16 tn .. of the remainder strip
  // the K loop in the form the tile needs: halo rows (conv tiles past the first), remainder rows
  auto run = [&](auto halo) {
    constexpr bool HV = decltype(halo)::value;
    if (rem)
      k_loop<BM, HV, R>(X, x_ld, W, M, N, K, m0, n0, n_rem0, lds, acc, hacc, racc, wr0, wc0, wm, wave, tn);
    else
      k_loop<BM, HV, false>(X, x_ld, W, M, N, K, m0, n0, n_rem0, lds, acc, hacc, racc, wr0, wc0, wm, wave, tn);
    if (rem && wave == tn / G::TM) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = m0 + 16 * tn + 4 * g + e, c = n_rem0 + m;
        if (r < M && c < N) Y[(size_t)r * y_ld + c] = f32_to_bf16(racc[e]);
      }
    }
  };
  uint16_t* out = reinterpret_cast<uint16_t*>(lds);
  if (!conv) {
    run(std::false_type{});
    stage_out<BM>(out, 0, acc, wr0, wc0);
    lds_sync();
    for (int e = threadIdx.x; e < BM * 16; e += GTHREADS) {
      const int r = e >> 4, c = (e & 15) * 8;
      if (m0 + r < M)
        *reinterpret_cast<uint4*>(Y + (size_t)(m0 + r) * y_ld + n0 + c) =
            *reinterpret_cast<const uint4*>(out + r * GBN + c);
    }
    return;
  }
  if constexpr (CONV) {
    // rows HALO + r of `out` hold tile row r (r >= -HALO): the halo rows, then the tile's own
    if (m0 > 0) {
      run(std::true_type{});
#pragma unroll
      for (int e = 0; e < 4; ++e) out[(4 * g + e) * GBN + 16 * wave + m] = f32_to_bf16(hacc[e]);
    } else {
      run(std::false_type{});
      // rows -3 .. -1: the history (oldest first), zeros without one
      if (threadIdx.x < 3 * GBN) {
        const int c = threadIdx.x % GBN, i = threadIdx.x / GBN;
        out[(HALO - 3 + i) * GBN + c] = hist_in != nullptr ? hist_in[(size_t)(n0 + c) * (CW - 1) + i] : (uint16_t)0;
      }
    }
    stage_out<BM>(out, HALO, acc, wr0, wc0);
    lds_sync();
    // conv + SiLU: thread t takes channels n0 + 2 (t % 64) .. + 1 over rows (t / 64) BM / 8 .. + BM / 8 - 1
    constexpr int RPW = BM / 8;
    const int cp = threadIdx.x & 63, r0 = wave * RPW;
    const int ch = n0 + 2 * cp;
    float w0[CW], w1[CW];
    {
      const uint2 a = *reinterpret_cast<const uint2*>(conv_w + (size_t)ch * CW);
      const uint2 b = *reinterpret_cast<const uint2*>(conv_w + (size_t)(ch + 1) * CW);
      w0[0] = __uint_as_float(a.x << 16), w0[1] = __uint_as_float(a.x & 0xffff0000u);
      w0[2] = __uint_as_float(a.y << 16), w0[3] = __uint_as_float(a.y & 0xffff0000u);
      w1[0] = __uint_as_float(b.x << 16), w1[1] = __uint_as_float(b.x & 0xffff0000u);
      w1[2] = __uint_as_float(b.y << 16), w1[3] = __uint_as_float(b.y & 0xffff0000u);
    }
    auto px = [&](int r) { return *reinterpret_cast<const uint32_t*>(out + (HALO + r) * GBN + 2 * cp); };
    uint32_t h0 = px(r0 - 3), h1 = px(r0 - 2), h2 = px(r0 - 1);
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
      const int r = r0 + rr;
      const uint32_t xv = px(r);
      float acc0 = fmaf(w0[0], __uint_as_float(h0 << 16), 0.f);
      float acc1 = fmaf(w1[0], __uint_as_float(h0 & 0xffff0000u), 0.f);
      acc0 = fmaf(w0[1], __uint_as_float(h1 << 16), acc0);
      acc1 = fmaf(w1[1], __uint_as_float(h1 & 0xffff0000u), acc1);
      acc0 = fmaf(w0[2], __uint_as_float(h2 << 16), acc0);
      acc1 = fmaf(w1[2], __uint_as_float(h2 & 0xffff0000u), acc1);
      acc0 = fmaf(w0[3], __uint_as_float(xv << 16), acc0);
      acc1 = fmaf(w1[3], __uint_as_float(xv & 0xffff0000u), acc1);
      // the conv rounded to bf16, then the activation (its result rounded by the store)
      const uint32_t pk = pack_bf16x2(acc0, acc1);
      const float y0 = silu_fast(__uint_as_float(pk << 16)), y1 = silu_fast(__uint_as_float(pk & 0xffff0000u));
      if (m0 + r < M) *reinterpret_cast<uint32_t*>(Y + (size_t)(m0 + r) * y_ld + ch) = pack_bf16x2(y0, y1);
      h0 = h1;
      h1 = h2;
      h2 = xv;
    }
    // the new history: the last 3 raw rows (rows before the first come from the old history)
    if (hist_out != nullptr && m0 <= M - 1 && M - 1 < m0 + BM && threadIdx.x < 3 * GBN) {
      const int c = threadIdx.x % GBN, i = threadIdx.x / GBN;
      hist_out[(size_t)(n0 + c) * (CW - 1) + i] = out[(HALO + M - (CW - 1) + i - m0) * GBN + c];
    }
  }
}

// Remainder columns [n_rem0, N) (fewer than 128): workgroups of 32 rows x 16 columns, K split over the 8 waves
// (wave w: row tile w % 2, K slice w / 2 of K / 4), the loads of 8 k-steps issued together, the four partial
// tiles of a row tile added in LDS in slice order.
__global__ __launch_bounds__(GTHREADS) void gemm_strip_kernel(const uint16_t* __restrict__ X, long x_ld,
                                                              const uint16_t* __restrict__ W, uint16_t* __restrict__ Y,
                                                              long y_ld, int M, int N, int K, int n_rem0) {
  __shared__ gf32x4 part[8][64];
  const int strips = (N - n_rem0 + 15) / 16;
  const int rb = blockIdx.x / strips, sc = blockIdx.x % strips;
  const int wave = wave_id(), l = threadIdx.x & 63, m = l & 15, g = l >> 4;
  const int rt = wave & 1, ks = wave >> 1, kq = K / 4;
  const int r0 = rb * 32 + rt * 16, c0 = n_rem0 + sc * 16;
  const uint16_t* xa = X + (size_t)min(r0 + m, M - 1) * x_ld + (size_t)ks * kq + 8 * g;
  const uint16_t* wb = W + (size_t)min(c0 + m, N - 1) * K + (size_t)ks * kq + 8 * g;
  gf32x4 acc = {0.f, 0.f, 0.f, 0.f};
  constexpr int U = 8;
  for (int k = 0; k < kq; k += 32 * U) {
    gbf16x8 a[U], b[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kk = min(k + 32 * u, kq - 32);  // (clamped: the loads stay unconditional)
      a[u] = *reinterpret_cast<const gbf16x8*>(xa + kk);
      b[u] = *reinterpret_cast<const gbf16x8*>(wb + kk);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (k + 32 * u < kq) acc = gmfma(a[u], b[u], acc);
  }
  part[wave][l] = acc;
  __syncthreads();
  if (ks == 0) {
    gf32x4 t = part[rt][l];
#pragma unroll
    for (int q = 1; q < 4; ++q) t += part[rt + 2 * q][l];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int r = r0 + 4 * g + e, c = c0 + m;
      if (r < M && c < N) Y[(size_t)r * y_ld + c] = f32_to_bf16(t[e]);
    }
  }
}

// n bf16 words of zeros (the history of a call without rows or old history).
__global__ void zero_u16_kernel(uint16_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// The GEMM kernels' dynamic LDS (above the default 64 KiB) is raised once per device and kernel (the first call on
// it); false when the device refuses.
template <int BM, bool CONV, bool R>
bool gemm_lds_ready() {
  static std::atomic<signed char> state[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  const signed char s = state[dev].load(std::memory_order_acquire);
  if (s != 0) return s > 0;
  const bool ok = hipFuncSetAttribute((const void*)gemm_kernel<BM, CONV, R>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      GemmCfg<BM>::LDS) == hipSuccess;
  if (!ok) (void)hipGetLastError();
  state[dev].store(ok ? 1 : -1, std::memory_order_release);
  return ok;
}

template <bool CONV>
int gemm_launch(const char* fn, const void* x, long x_ld, const void* w, void* y, long y_ld, int M, int N, int K,
                const void* conv_w, int C, const void* hist_in, void* hist_out, hipStream_t s) {
  const int n_full_cols = N / GBN, n_rem0 = n_full_cols * GBN;
  bool strip = n_rem0 < N;
  if (n_full_cols > 0) {
    // 128-row tiles, two workgroups a CU: measured faster than 256-row tiles at one a CU for every shape of the
    // layer (in_proj 4096 x 2056 x 1024: 22.3 against 24.7 us; 4096 x 2048 x 1024: 21.1 against 24.1 us), as one
    // workgroup's epilogue (the conv's VALU work) runs beside the other's MFMAs. A remainder of at most 16
    // columns is formed by the tiles when their column count covers a row block in 16-row pieces.
#define ZGDN_GEMM(BMV, RV)                                                                                          \
  do {                                                                                                              \
    if (!gemm_lds_ready<BMV, CONV, RV>()) return fail(ZGDN_EHIP, "%s: the device refused the GEMM's LDS", fn);     \
    const int tm = (M + (BMV) - 1) / (BMV);                                                                        \
    hipLaunchKernelGGL((gemm_kernel<BMV, CONV, RV>), dim3(tm * n_full_cols), dim3(GTHREADS), GemmCfg<BMV>::LDS, s, \
                       (const uint16_t*)x, x_ld, (const uint16_t*)w, (uint16_t*)y, y_ld, M, N, K, tm, n_full_cols, \
                       (const uint16_t*)conv_w, C, (const uint16_t*)hist_in, (uint16_t*)hist_out);                 \
  } while (0)
    const bool fold = strip && N - n_rem0 <= 16 && 16 * n_full_cols >= 128;
    if (fold)
      ZGDN_GEMM(128, true);
    else
      ZGDN_GEMM(128, false);
#undef ZGDN_GEMM
    strip = strip && !fold;
  }
  if (strip) {
    const int strips = (N - n_rem0 + 15) / 16;
    hipLaunchKernelGGL(gemm_strip_kernel, dim3(((M + 31) / 32) * strips), dim3(GTHREADS), 0, s, (const uint16_t*)x,
                       x_ld, (const uint16_t*)w, (uint16_t*)y, y_ld, M, N, K, n_rem0);
  }
  return check_launch(fn);
}

int gemm_check(const char* fn, const void* x, long x_ld, const void* w, const void* y, long y_ld, int M, int N, int K,
               int dtype) {
  if (dtype != ZGDN_BF16) return fail(ZGDN_EUNSUPPORTED, "%s: bf16 only (dtype %d)", fn, dtype);
  if (M < 0 || N < 1 || K < 1) return fail(ZGDN_EINVAL, "%s: bad sizes M=%d N=%d K=%d", fn, M, N, K);
  if (M > 0 && (!x || !w || !y)) return fail(ZGDN_EINVAL, "%s: null pointer", fn);
  // (K a multiple of 128: whole K blocks, and whole k-steps in each quarter of K the strip kernel splits)
  if (K % (2 * GK) || N % 8 || x_ld < K || y_ld < N || x_ld % 8 || y_ld % 8 ||
      ((uintptr_t)x | (uintptr_t)w | (uintptr_t)y) % 16)
    return fail(ZGDN_EINVAL, "%s: K=%d (a multiple of %d), N=%d and row strides x=%ld y=%ld (multiples of 8 "
                "elements, >= K / N) from 16-byte aligned bases", fn, K, 2 * GK, N, x_ld, y_ld);
  if ((long)M * x_ld * 2 >= (1L << 32) || (long)N * K * 2 >= (1L << 32))
    return fail(ZGDN_EUNSUPPORTED, "%s: operands of 4 GiB or more", fn);
  return ZGDN_OK;
}

}  // namespace
}  // namespace zgdn

extern "C" int zgdn_gemm_nt(const void* x, long x_ld, const void* w, void* y, long y_ld, int M, int N, int K,
                            int dtype, void* stream) {
  using namespace zgdn;
  const char* fn = "zgdn_gemm_nt";
  const int st = gemm_check(fn, x, x_ld, w, y, y_ld, M, N, K, dtype);
  if (st != ZGDN_OK || M == 0) return st;
  return gemm_launch<false>(fn, x, x_ld, w, y, y_ld, M, N, K, nullptr, 0, nullptr, nullptr, (hipStream_t)stream);
}

extern "C" int zgdn_in_proj_conv(const void* x, long x_ld, const void* w, void* y, long y_ld, int M, int N, int K,
                                 const void* conv_weight, int C, const void* hist_in, void* hist_out, int dtype,
                                 void* stream) {
  using namespace zgdn;
  const char* fn = "zgdn_in_proj_conv";
  int st = gemm_check(fn, x, x_ld, w, y, y_ld, M, N, K, dtype);
  if (st != ZGDN_OK) return st;
  if (C < GBN || C % GBN || C > N || conv_weight == nullptr)
    return fail(ZGDN_EINVAL, "%s: conv channels C=%d (a multiple of %d, <= N=%d) and the conv weight", fn, C, GBN, N);
  if (hist_in != nullptr && hist_in == hist_out)
    return fail(ZGDN_EINVAL, "%s: the new history may not overwrite the old one in place", fn);
  if (((uintptr_t)conv_weight) % 8) return fail(ZGDN_EINVAL, "%s: conv weight not 8-byte aligned", fn);
  if (M == 0) {  // no rows: the history passes through (zeros without one; a fill kernel, not a memset node)
    if (hist_out == nullptr) return ZGDN_OK;
    if (hist_in != nullptr) {
      const hipError_t e = hipMemcpyAsync(hist_out, hist_in, (size_t)C * (CW - 1) * 2, hipMemcpyDeviceToDevice,
                                          (hipStream_t)stream);
      if (e != hipSuccess) return fail(ZGDN_EHIP, "%s: %s", fn, hipGetErrorString(e));
      return ZGDN_OK;
    }
    const int n = C * (CW - 1);
    hipLaunchKernelGGL(zero_u16_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, (uint16_t*)hist_out, n);
    return check_launch(fn);
  }
  return gemm_launch<true>(fn, x, x_ld, w, y, y_ld, M, N, K, conv_weight, C, hist_in, hist_out, (hipStream_t)stream);
}
