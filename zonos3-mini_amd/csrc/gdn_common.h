// Shared device helpers for the gated-DeltaNet kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "zonos3_gdn.h"

namespace zgdn {

// ------------------------------------------------------------------------------------------------ bf16 storage

struct bf16 {
  uint16_t bits;
};

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// float -> bf16, round to nearest even (one v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// Two floats -> two bf16 packed in one word (a in the low half), one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

template <typename T>
struct io;

template <>
struct io<float> {
  __device__ __forceinline__ static float load(const float* p) { return *p; }
  __device__ __forceinline__ static void store(float* p, float x) { *p = x; }
  // Four consecutive elements as floats.
  __device__ __forceinline__ static float4 load4(const float* p) { return *reinterpret_cast<const float4*>(p); }
  __device__ __forceinline__ static void store4(float* p, float4 x) { *reinterpret_cast<float4*>(p) = x; }
};

template <>
struct io<bf16> {
  __device__ __forceinline__ static float load(const bf16* p) { return bf16_to_f32(p->bits); }
  __device__ __forceinline__ static void store(bf16* p, float x) { p->bits = f32_to_bf16(x); }
  __device__ __forceinline__ static float4 load4(const bf16* p) {
    uint2 w = *reinterpret_cast<const uint2*>(p);
    return make_float4(__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u),
                       __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xffff0000u));
  }
  __device__ __forceinline__ static void store4(bf16* p, float4 x) {
    *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf16x2(x.x, x.y), pack_bf16x2(x.z, x.w));
  }
};

// --------------------------------------------------------------------------------------- cross-lane reductions

// DPP move of a float within a row of 16 lanes (every source lane is valid for the patterns used here).
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

constexpr int DPP_QUAD_XOR1 = 0xB1;       // quad_perm(1,0,3,2)
constexpr int DPP_QUAD_XOR2 = 0x4E;       // quad_perm(2,3,0,1)
constexpr int DPP_ROW_HALF_MIRROR = 0x141;  // lane i <-> 7-i within each 8-lane half row
constexpr int DPP_ROW_MIRROR = 0x140;     // lane i <-> 15-i within each 16-lane row

// Sum over aligned groups of N lanes (N = 4, 8 or 16); every lane of a group receives the group sum.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(N == 4 || N == 8 || N == 16, "group of 4, 8 or 16 lanes");
  x += dpp<DPP_QUAD_XOR1>(x);
  x += dpp<DPP_QUAD_XOR2>(x);
  if constexpr (N >= 8) x += dpp<DPP_ROW_HALF_MIRROR>(x);
  if constexpr (N >= 16) x += dpp<DPP_ROW_MIRROR>(x);
  return x;
}

// Sum over all 64 lanes of a wave (result valid in every lane): the row sums by DPP, then rows 0 + 1 and 2 + 3,
// then the two halves, with the gfx950 permlane swaps (each lane gets its partner row's, then half's, value in
// registers, no LDS round trip). The swaps pair lane l with l ^ 16, then l ^ 32, as lane-xor steps would, so
// every lane's sum is the same to the bit.
__device__ __forceinline__ float wave_sum(float x) {
  x = group_sum<16>(x);
  auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

// This wave's index in the workgroup as a wave-uniform (scalar) value: indexing by it then takes scalar
// loads and branches (threadIdx.x >> 6 alone is a per-lane value to the compiler).
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Maximum over all 64 lanes of a wave (result valid in every lane): DPP within each row of 16 lanes, then the
// gfx950 permlane swaps (each lane gets its partner row's, then half's, value in registers).
__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, dpp<DPP_QUAD_XOR1>(x));
  x = fmaxf(x, dpp<DPP_QUAD_XOR2>(x));
  x = fmaxf(x, dpp<DPP_ROW_HALF_MIRROR>(x));
  x = fmaxf(x, dpp<DPP_ROW_MIRROR>(x));
  auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
  p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}

// ---------------------------------------------------------------------------------------- packed sequences

// Token range [bos, eos) of packed sequence s (cu_seqlens int32 [n + 1]), clamped into [0, T]: a table that
// decreases or runs past the T tokens of the batch gives empty or shortened ranges, so no kernel reads or
// writes a token row outside the batch. (The host layer rejects such tables wherever it holds them.)
__device__ __forceinline__ void seq_bounds(const int32_t* cu, int s, int T, int& bos, int& eos) {
  bos = min(max(cu[s], 0), T);
  eos = min(max(cu[s + 1], bos), T);
}

// ------------------------------------------------------------------------------------------ buffer resources

// Buffer resource of a raw byte range (no stride, no swizzle; the 32-bit data format gfx9 takes for untyped
// accesses): stores at byte offsets past `bytes` are dropped and loads there read zero. Formed in scalar
// registers, so that loads and stores through it take a per-lane offset and no 64-bit vector address
// arithmetic, and rows past a range's end need no per-lane condition (a store under a lane condition makes
// the compiler wait for every outstanding load at the join).
typedef __amdgpu_buffer_rsrc_t Rsrc;
__device__ __forceinline__ Rsrc raw_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// ------------------------------------------------------------------------------------------ chunked prefill

constexpr int CHUNK_LEN = 64;  // tokens per chunk of the chunked (WY / UT form) prefill

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
    int bos, eos;
    seq_bounds(cu, s, T, bos, eos);
    if (j >= (eos - bos + CHUNK_LEN - 1) / CHUNK_LEN) {  // past the sequence's chunks
      r.t0 = 0;
      r.len = 0;
      return r;
    }
    r.t0 = bos + j * CHUNK_LEN;
    r.len = min(CHUNK_LEN, eos - r.t0);
  } else {
    const int nt = (T + CHUNK_LEN - 1) / CHUNK_LEN;
    const int b = c / nt, j = c % nt;
    r.t0 = b * T + j * CHUNK_LEN;
    r.len = min(CHUNK_LEN, T - j * CHUNK_LEN);
  }
  return r;
}

// First chunk (in the canonical table order: sequence by sequence, chunk by chunk) and token range of packed
// sequence `seq` (cu != nullptr), or of batch row `seq` of an unpacked B x T batch.
__device__ __forceinline__ void seq_chunks(const int32_t* cu, int seq, int T, int& c0, int& bos, int& len) {
  if (cu != nullptr) {
    int eos;
    seq_bounds(cu, seq, T, bos, eos);
    len = eos - bos;
    c0 = 0;
    for (int s = 0; s < seq; ++s) {
      int sb, se;
      seq_bounds(cu, s, T, sb, se);
      c0 += (se - sb + CHUNK_LEN - 1) / CHUNK_LEN;
    }
  } else {
    bos = seq * T;
    len = T;
    c0 = seq * ((T + CHUNK_LEN - 1) / CHUNK_LEN);
  }
}

// Elements between consecutive tokens of q, k, v and of g / beta (a token's heads are contiguous in each), so
// that the kernel reads column slices of wider rows (the conv output, the input projection) in place;
// beta_sigmoid: beta holds the raw input b and the kernel takes sigmoid(b) (in fp32).
struct RowStrides {
  long q, k, v, gb;
  int beta_sigmoid;
};

// -------------------------------------------------------------------------------------------------- math

__device__ __forceinline__ float softplus(float x) { return x > 20.f ? x : log1pf(__expf(x)); }
__device__ __forceinline__ float sigmoid(float x) { return 1.f / (1.f + __expf(-x)); }
__device__ __forceinline__ float silu(float x) { return x / (1.f + __expf(-x)); }
// x * sigmoid(x) with the hardware reciprocal (v_rcp_f32, ~1 ulp) in place of the division: a few
// instructions instead of the division's ten; for results that are rounded to bf16 or compared at 1e-5.
__device__ __forceinline__ float silu_fast(float x) { return x * __builtin_amdgcn_rcpf(1.f + __expf(-x)); }

}  // namespace zgdn

// ------------------------------------------------------------------------------------------- host-side errors

namespace zgdn {
// Records a message for zgdn_last_error() and returns `code`.
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);

// The fp32-arithmetic chunked path (gdn_chunk_f32.hip): workspace bytes per (chunk, value head) item at head
// size D, and the forward behind zgdn_chunk_fwd for fp32 q/k/v and for 64-wide heads (arguments checked there).
size_t chunk32_item_bytes(int D);
int chunk32_fwd(const char* fn, const void* q, const void* k, const void* v, int qkv_dtype, const void* g,
                const void* beta, int gb_dtype, const float* A_log, const float* dt_bias, int qk_l2norm,
                const float* s_in, float* s_out, void* o, const int32_t* cu, const int32_t* chunk_idx, int N,
                int n_chunks, int T, int Hk, int Hv, int D, float scale, const RowStrides& rs, void* workspace,
                hipStream_t s);
}  // namespace zgdn
