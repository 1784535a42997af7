// Block Attention Residual (AttnRes) routing kernels for gfx950 (CDNA4).
//
// One routing point mixes, for every token independently, S depth sources
// (committed block summaries plus the running partial block) of width d:
//
//   qw       = query * gain                            (llama.py:630)
//   inv_rms  = rsqrt(mean_d(x_s^2) + eps)              (llama.py:640)
//   logit_s  = (x_s . qw) * inv_rms_s                  (llama.py:641)
//   w        = softmax over s of logit                 (llama.py:642-643)
//   out      = sum_s w_s * x_s   (raw, un-normalised)  (llama.py:644)
//
// With one query the work is a GEMV per token at ~2 flop/byte, bound by HBM.
// The kernel families (each row-block of a source is a separate pointer; no
// stacked copy is needed):
//
//   * attnres_stream_*  one wave per token row (prefill; the hot path).  A
//     lane holds 16-byte chunks l, l+64, ..., so each wave-wide load is 1 KiB
//     contiguous.  The wave's (token, source) items flow through a two-slot
//     register pipeline (the next row is requested once the current one has
//     arrived, before it is processed: one row per wave in flight); per
//     source: sum(x^2) and x.qw, one DPP wave reduction each, then an online
//     softmax with the rescale folded into the accumulating FMA.  Finished
//     output rows are staged in LDS and stored in batches per wave; one
//     workgroup of four waves per CU (three for 8 KiB rows).
//   * attnres_route_*   one workgroup per token row (decode, few rows, Q > 1
//     queries, the fused arena modes).  Thread i owns chunks i, i+blockDim,
//     ...; all S source chunks are loaded at once, partial sums are reduced
//     per wave by a transposing permlane/DPP tree and across waves through
//     one double-buffered LDS exchange, and the softmax is exact (two-pass
//     over registers).  The _qg instances batch Q queries (staged in LDS) and
//     mix sources on the matrix cores (v_mfma_f32_4x4x4_16b_bf16, weights as
//     bf16 hi + lo), since Q queries turn the mix into a small product.
//   * attnres_merge_*   the phase-2 merge of a running block into a phase-1
//     result: attnres_merge_stream_* one wave per row (the partial and inter
//     rows stream one row per pipeline slot), attnres_merge_<p>_<i>_v* one
//     workgroup per row.
//   * attnres_route_bwd_* / _mq_ / _mqg_ / _dqw* / merge_bwd / reduce_dqw*:
//     the backward of routing and merge (source, query and gain gradients;
//     the query gradient summed over rows in a fixed order), the batched-
//     query forms again on the matrix cores.  attnres_route_bwd_stream_* is
//     the routing backward with one wave per token row (the training shapes'
//     bf16 rows of 6 KiB): the row's G and source rows stream through the
//     same two-slot pipeline, the source rows are kept in registers, and the
//     gradient rows are stored whole after the row's softmax; its _defer
//     instances leave the committed blocks' gradients as per-token
//     coefficients, which attnres_route_bwd_gather_seg_* sum over the
//     training loop's points on the matrix cores.
//
// S is a template parameter of the row-per-workgroup kernels (register arrays
// stay in VGPRs) and a runtime argument of the streaming ones; the last slot
// can be formed in-kernel from a sublayer delta (fused partial accumulate /
// block commit for the decode and arena paths).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "attnres_params.h"

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

namespace {

// ---------------------------------------------------------------- helpers --

// Reinterpret one 32-bit lane as fp32.  Taking the word by value matters:
// __builtin_bit_cast applied directly to an ext_vector element lvalue
// (bit_cast<float>(v[i])) is lowered as a cast of element 0 by this compiler.
__device__ __forceinline__ float as_f32(uint32_t u) { return __builtin_bit_cast(float, u); }
__device__ __forceinline__ uint32_t as_u32(float f) { return __builtin_bit_cast(uint32_t, f); }

__device__ __forceinline__ float bf_lo(uint32_t u) { return __builtin_bit_cast(float, u << 16); }
__device__ __forceinline__ float bf_hi(uint32_t u) { return __builtin_bit_cast(float, u & 0xffff0000u); }

// Two fp32 -> packed bf16 pair, round-to-nearest-even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  bf16x2 r = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ float round_bf16(float v) { return (float)(__bf16)v; }

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c,
                                         false);
}

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// v_mfma_f32_4x4x4_16b_bf16: sixteen independent 4x4x4 products per wave,
// block b on lanes 4b..4b+3.  Lane 4b+i supplies row i of A and lane 4b+j
// column j of B (four bf16 along k each, packed two per word); lane 4b+j
// receives column j of D, element i holding D[i][j] = C[i][j] + sum_k
// A[i][k] B[k][j] in fp32.
__device__ __forceinline__ f32x4 mfma_4x4x4(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(i16x4, a), __builtin_bit_cast(i16x4, b), c, 0,
                                                0, 0);
}

// A wave-uniform 64-bit integer kept in SGPRs.
__device__ __forceinline__ int64_t uniform_i64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)(uint64_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// A wave-uniform float kept in an SGPR.
__device__ __forceinline__ float uniform_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(uint32_t, v)));
}

// A wave-uniform address held in SGPRs (the value is the same in every lane).
__device__ __forceinline__ const char* uniform_ptr(uint64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const char*>(((uint64_t)hi << 32) | lo);
}

template <typename T>
__device__ __forceinline__ T ldg(const void* p) {
  return *reinterpret_cast<const T*>(p);
}

// Source rows are read exactly once, so they are loaded with the
// non-temporal hint; on MI355X this raised the routing kernels from ~5.0 to
// ~5.7 TB/s at S=8.  Output rows are written with system-scope (sc1)
// buffer stores, which measured 3.5-5% faster than default or non-temporal
// stores in this read-heavy mix.  Build switches:
#ifndef ATTNRES_NT_LOADS
#define ATTNRES_NT_LOADS 1
#endif
#ifndef ATTNRES_NT_STORES
#define ATTNRES_NT_STORES 0
#endif
#ifndef ATTNRES_STORE_CPOL
#define ATTNRES_STORE_CPOL 16  // buffer-store cache policy: 16 = sc1
#endif
#ifndef ATTNRES_LOAD_CPOL
#define ATTNRES_LOAD_CPOL -1  // -1: global loads (nt per ATTNRES_NT_LOADS); >= 0: buffer loads with this policy
#endif

// A wave-uniform fp32 read through the scalar data cache (s_load): its wait
// counts with the LDS operations, not with the vector loads in flight.
__device__ __forceinline__ float ld_scalar_f32(const float* p) {
  return *(const __attribute__((address_space(4))) float*)(p);
}

// Zero that the compiler cannot fold, computed from v: adding it to the next
// load's offset makes that load wait until v has arrived.  The streaming
// kernels pass the last register of the row just loaded, so a wave requests
// its next row only once the current one is in (one row per wave in flight
// while the wave works on it; loads return in order, so the last register
// arriving means the whole row has).
__device__ __forceinline__ uint32_t arrival_zero(uint32_t v) {
  uint32_t z;
  asm volatile("v_and_b32 %0, 0, %1" : "=v"(z) : "v"(v));
  return z;
}

// Load through an explicitly global pointer: a generic (flat) load would also
// count against the LDS wait counter and serialise with LDS reads.
template <typename T>
__device__ __forceinline__ T ldg_global(const char* p) {
  const __attribute__((address_space(1))) T* g = (const __attribute__((address_space(1))) T*)(p);
#if ATTNRES_NT_LOADS
  return __builtin_nontemporal_load(g);
#else
  return *g;
#endif
}
template <typename T>
__device__ __forceinline__ void stg(void* p, T v) {
  *reinterpret_cast<T*>(p) = v;
}

// Output rows: a buffer resource over one row (base in SGPRs, byte range =
// the row, so a store outside it is dropped by the hardware) and raw buffer
// stores carrying the cache policy above.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(char* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(base, 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 ld_row(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, ATTNRES_LOAD_CPOL < 0 ? 0 : ATTNRES_LOAD_CPOL);
}
__device__ __forceinline__ void st_row(__amdgpu_buffer_rsrc_t r, uint32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, ATTNRES_STORE_CPOL);
}
__device__ __forceinline__ void st_row(__amdgpu_buffer_rsrc_t r, uint32_t off, u32x2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, ATTNRES_STORE_CPOL);
}
// Non-temporal stores: the routing backward kernels (the 3B backward sweep
// 2.4% faster, the 8B one 0.5%), the serving backward (merge and batched
// backward, 2.4%), the arena's fused block steps (2%) and the deferred
// gradient sums (2-3% in the training step) measured faster with them; the
// list and batched-query forward kernels and the fused step writing its
// partial to a new buffer 1.5-9% slower.
__device__ __forceinline__ void st_row_nt(__amdgpu_buffer_rsrc_t r, uint32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, 2);
}
__device__ __forceinline__ void st_row_nt(__amdgpu_buffer_rsrc_t r, uint32_t off, u32x2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, 2);
}

// Stores hidden from the compiler's wait-count model.  One counter (vmcnt)
// covers vector loads and stores, and the compiler, which cannot order a
// pending store against a pending load, waits for a loaded register with
// vmcnt(0) whenever one of its stores may be in flight: every prefetched row
// drains.  Loads complete in issue order, so a wait until no more loads are
// outstanding than were issued after the one awaited proves that load
// complete whatever stores are in flight as well (they only lengthen the
// wait); with the stores issued from inline assembly the compiler counts
// loads alone and its waits keep the later loads in flight (kernels that
// keep several loads in flight across their stores).  The s_nop covers the
// store-data hazard of a VALU write right after the store.
__device__ __forceinline__ void st_row_nt_hidden(__amdgpu_buffer_rsrc_t r, uint32_t off, u32x4 v) {
  asm volatile("buffer_store_dwordx4 %0, %1, %2, 0 offen nt\n\ts_nop 1" : : "v"(v), "v"(off), "s"(r) : "memory");
}
__device__ __forceinline__ void st_f32_hidden(float* p, float v) {
  asm volatile("global_store_dword %0, %1, off\n\ts_nop 1" : : "v"(p), "v"(v) : "memory");
}

template <typename T>
__device__ __forceinline__ void stg_global(char* p, T v) {
  __attribute__((address_space(1))) T* g = (__attribute__((address_space(1))) T*)(p);
#if ATTNRES_NT_STORES
  __builtin_nontemporal_store(v, g);
#else
  *g = v;
#endif
}

// In-place accumulator updates on one 32-bit source word.  The tied "+v"
// operands keep every fp32 accumulator in one register across the softmax
// branches (written as plain fmaf, the compiler renames the accumulator row
// per branch and copies at the joins, doubling its register footprint), and
// the bf16 -> fp32 unpack happens inside, so it cannot be hoisted above the
// branch into a second copy of the row.
//   rescale_add: acc = acc * c + x        add_scaled: acc = acc + p * x
__device__ __forceinline__ void acc_rescale_add_bf16(float& lo, float& hi, uint32_t w, float c) {
  float t;
  asm("v_lshlrev_b32 %2, 16, %3\n\t"
      "v_fma_f32 %0, %0, %4, %2\n\t"
      "v_and_b32 %2, 0xffff0000, %3\n\t"
      "v_fma_f32 %1, %1, %4, %2"
      : "+v"(lo), "+v"(hi), "=&v"(t)
      : "v"(w), "v"(c));
}
__device__ __forceinline__ void acc_add_scaled_bf16(float& lo, float& hi, uint32_t w, float p) {
  float t;
  asm("v_lshlrev_b32 %2, 16, %3\n\t"
      "v_fmac_f32 %0, %4, %2\n\t"
      "v_and_b32 %2, 0xffff0000, %3\n\t"
      "v_fmac_f32 %1, %4, %2"
      : "+v"(lo), "+v"(hi), "=&v"(t)
      : "v"(w), "v"(p));
}
// The scale c / p comes straight from v_exp_f32, a transcendental op whose
// result a VALU may only read after one wait state.  The compiler inserts
// that wait for its own code but not inside inline asm, so every asm block
// above starts with an instruction that does not read c / p.  The fp32
// forms below have no unpack to put first and stay plain C.
__device__ __forceinline__ void acc_rescale_add_f32(float& acc, uint32_t w, float c) {
  acc = __builtin_fmaf(acc, c, as_f32(w));
}
__device__ __forceinline__ void acc_add_scaled_f32(float& acc, uint32_t w, float p) {
  acc = __builtin_fmaf(as_f32(w), p, acc);
}
__device__ __forceinline__ void acc_zero(float& acc) { asm("v_mov_b32 %0, 0" : "+v"(acc)); }

// One DPP step: v + v[permuted lane], restricted to the rows in ROW_MASK.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
  const int t = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF, false);
  return v + __builtin_bit_cast(float, t);
}

// Sum over the 64 lanes of a wave; the full sum lands in lane 63.
//   quad_perm[1,0,3,2], quad_perm[2,3,0,1]  -> quad sums
//   row_half_mirror, row_mirror             -> row (16-lane) sums in every lane
//   row_bcast:15 (rows 1,3), row_bcast:31 (rows 2,3) -> lane 63 holds the total
__device__ __forceinline__ float wave_sum_to_lane63(float v) {
  v = dpp_add<0xB1, 0xF>(v);
  v = dpp_add<0x4E, 0xF>(v);
  v = dpp_add<0x141, 0xF>(v);
  v = dpp_add<0x140, 0xF>(v);
  v = dpp_add<0x142, 0xA>(v);
  v = dpp_add<0x143, 0xC>(v);
  return v;
}

// Elements of a 16-byte chunk as fp32.
template <bool BF16>
struct Chunk;

template <>
struct Chunk<true> {  // 8 x bf16
  static constexpr int VEC = 8;
  static constexpr int BYTES = 2;
  __device__ __forceinline__ static float elem(const u32x4& c, int e) {
    const uint32_t w = c[e >> 1];
    return (e & 1) ? bf_hi(w) : bf_lo(w);
  }
};

template <>
struct Chunk<false> {  // 4 x fp32
  static constexpr int VEC = 4;
  static constexpr int BYTES = 4;
  __device__ __forceinline__ static float elem(const u32x4& c, int e) { return as_f32(c[e]); }
};

// Load VEC consecutive parameter elements (bf16 or fp32) as fp32.
template <int VEC>
__device__ __forceinline__ void load_param(const void* base, int64_t elem_off, bool bf16, float (&v)[VEC]) {
  if (bf16) {
    const uint16_t* p = reinterpret_cast<const uint16_t*>(base) + elem_off;
#pragma unroll
    for (int e = 0; e < VEC; ++e) v[e] = __builtin_bit_cast(float, (uint32_t)p[e] << 16);
  } else {
    const float* p = reinterpret_cast<const float*>(base) + elem_off;
#pragma unroll
    for (int e = 0; e < VEC; ++e) v[e] = p[e];
  }
}

// qw chunk = query[q] * gain, rounded to the parameter dtype the way the
// reference's `query * norm.weight` is (llama.py:630; serve.py:89-91).
template <int VEC>
__device__ __forceinline__ void load_qw(const attnres_route_params& P, int q, int chunk, float (&qw)[VEC]) {
  const int64_t off = (int64_t)chunk * VEC;
  load_param<VEC>(P.query, (int64_t)q * P.d + off, P.param_bf16, qw);
  if (P.gain != nullptr) {
    float g[VEC];
    load_param<VEC>(P.gain, off, P.param_bf16, g);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float prod = qw[e] * g[e];
      qw[e] = P.param_bf16 ? round_bf16(prod) : prod;
    }
  }
}

// A parameter chunk (VEC elements, bf16 or fp32 by a runtime flag) loaded
// packed; converted with param_elem after every load of the prologue has been
// issued, so the loads share one wait.
template <int VEC>
struct ParamRaw {
  u32x4 w[VEC == 8 ? 2 : 1];
};
template <int VEC>
__device__ __forceinline__ void load_param_raw(const void* base, int chunk, bool bf16, ParamRaw<VEC>& r) {
  const char* b = reinterpret_cast<const char*>(base);
  if (bf16) {
    if constexpr (VEC == 8) {
      r.w[0] = ldg_global<u32x4>(b + (int64_t)chunk * 16);
      r.w[1] = u32x4{0, 0, 0, 0};
    } else {
      const u32x2 t = ldg_global<u32x2>(b + (int64_t)chunk * 8);
      r.w[0] = u32x4{t[0], t[1], 0, 0};
    }
  } else {
#pragma unroll
    for (int h = 0; h < VEC / 4; ++h) r.w[h] = ldg_global<u32x4>(b + ((int64_t)chunk * VEC + 4 * h) * 4);
  }
}
template <int VEC>
__device__ __forceinline__ float param_elem(const ParamRaw<VEC>& r, int e, bool bf16) {
  if (bf16) {
    const uint32_t w = r.w[0][e >> 1];
    return (e & 1) ? bf_hi(w) : bf_lo(w);
  }
  return as_f32(r.w[e >> 2][e & 3]);
}

// ------------------------------------------------ wave reductions --

// Exchange lanes 32..63 of a with lanes 0..31 of b (v_permlane32_swap), and
// the odd 16-lane rows of a with the even rows of b (v_permlane16_swap).  The
// leading s_nop covers the VALU-write -> permlane-read hazard.  Inline asm:
// this compiler's __builtin_amdgcn_permlane{16,32}_swap return the first
// register for both results.
__device__ __forceinline__ void swap_halves32(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap_rows16(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_max(float v) {
  const int t = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF, false);
  return __builtin_fmaxf(v, __builtin_bit_cast(float, t));
}

// Max / sum over aligned segments of SEG (8 or 16) lanes, result in every
// lane of the segment: quad_perm[1,0,3,2], quad_perm[2,3,0,1],
// row_half_mirror (8 lanes), row_mirror (16 lanes).
template <int SEG>
__device__ __forceinline__ float seg_max(float v) {
  v = dpp_max<0xB1, 0xF>(v);
  v = dpp_max<0x4E, 0xF>(v);
  v = dpp_max<0x141, 0xF>(v);
  if constexpr (SEG == 16) v = dpp_max<0x140, 0xF>(v);
  return v;
}
template <int SEG>
__device__ __forceinline__ float seg_sum(float v) {
  v = dpp_add<0xB1, 0xF>(v);
  v = dpp_add<0x4E, 0xF>(v);
  v = dpp_add<0x141, 0xF>(v);
  if constexpr (SEG == 16) v = dpp_add<0x140, 0xF>(v);
  return v;
}

// Sum over the 64 lanes of each of NP = 4*H2 values part[0..NP), written to
// red_row[v] for every v < NP by the first lane of each 16-lane row.  Two
// swap rounds leave register j of row rho holding value
// j + (rho & 1) * H2 + (rho >> 1) * 2 * H2 (summed over 4 lanes); four DPP
// steps finish the 16-lane row sums.
template <int H2>
__device__ __forceinline__ void wave_reduce_to_lds(float (&part)[4 * H2], float* red_row, int lane) {
  constexpr int H1 = 2 * H2;
  float r1[H1];
#pragma unroll
  for (int j = 0; j < H1; ++j) {
    float a = part[j], b = part[j + H1];
    swap_halves32(a, b);
    r1[j] = a + b;
  }
  float r2[H2];
#pragma unroll
  for (int j = 0; j < H2; ++j) {
    float a = r1[j], b = r1[j + H2];
    swap_rows16(a, b);
    r2[j] = seg_sum<16>(a + b);
  }
  const int rho = lane >> 4;
  if ((lane & 15) == 0) {
    float* dst = red_row + (rho & 1) * H2 + (rho >> 1) * H1;
#pragma unroll
    for (int j = 0; j < H2; ++j) dst[j] = r2[j];
  }
}

// ------------------------------------------------------------ route body --

// S     : number of active sources (0 writes NaN, as softmax over no sources)
// V     : 16-byte chunks per thread per source row
// BF16  : sources (and delta) are bf16, else fp32
// QDOT2 : bf16 sources and bf16-exact qw: the dot uses v_dot2c_f32_bf16
// MULTIQ: num_queries >= 1 queries share the loaded rows (phase-1 batching)
template <int S, int V, bool BF16, bool QDOT2, bool MULTIQ>
__device__ __forceinline__ void route_body(const attnres_route_params& P) {
  using C = Chunk<BF16>;
  constexpr int VEC = C::VEC;
  constexpr int NV = 2 * S;                  // sum(x^2) and x.qw per source
  constexpr int NP = ((NV + 3) / 4) * 4 > 0 ? ((NV + 3) / 4) * 4 : 4;  // padded for the reduction
  constexpr int SEG = S <= 8 ? 8 : 16;       // lanes of the depth softmax
  __shared__ float red[2][ATTNRES_KMAX_WAVES][NP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int block = P.block;
  const int nwaves = (block + 63) >> 6;
  const int nq = MULTIQ ? P.num_queries : 1;
  const int ls = lane % SEG;  // the source of this lane in the softmax
  const bool slot = ls < S;

  int chunk[V];
  bool ok[V];
#pragma unroll
  for (int k = 0; k < V; ++k) {
    chunk[k] = tid + k * block;
    ok[k] = chunk[k] < P.nchunk;
  }

  // Pseudo-query chunks, kept in registers across the token loop (Q == 1).
  float qwf[V][VEC];
  uint32_t qwb[V][VEC / 2];
  auto set_qw = [&](int k, const float (&t)[VEC]) {
    if constexpr (QDOT2) {
#pragma unroll
      for (int e = 0; e < VEC / 2; ++e) qwb[k][e] = pack_bf16(t[2 * e], t[2 * e + 1]);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) qwf[k][e] = t[e];
    }
  };
  auto fetch_qw = [&](int q) {  // multi-query: query q of the batch
#pragma unroll
    for (int k = 0; k < V; ++k) {
      float t[VEC];
      if (ok[k]) {
        load_qw<VEC>(P, q, chunk[k], t);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) t[e] = 0.f;
      }
      set_qw(k, t);
    }
  };
  const int64_t row_bytes_ld = P.src_ld * C::BYTES;
  // One token row of sources (and, fused, of the delta) in registers.  The
  // first row is requested before the parameters, so a workgroup that owns a
  // single row (decode) waits for memory once, not once per dependent load.
  constexpr int SX = S > 0 ? S : 1;
  u32x4 x[SX][V];
  u32x4 dvr[V];
  auto load_row = [&](int64_t t) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const char* row = reinterpret_cast<const char*>(P.src[s]) + t * row_bytes_ld;
#pragma unroll
      for (int k = 0; k < V; ++k) {
        if (s == S - 1 && P.mode == ATTNRES_MODE_SET) {
          x[s][k] = u32x4{0, 0, 0, 0};
        } else {
          x[s][k] = ok[k] ? ldg_global<u32x4>(row + (int64_t)chunk[k] * 16) : u32x4{0, 0, 0, 0};
        }
      }
    }
    if (S > 0 && P.mode != ATTNRES_MODE_PLAIN) {
      const char* drow = reinterpret_cast<const char*>(P.delta) + t * P.delta_ld * C::BYTES;
#pragma unroll
      for (int k = 0; k < V; ++k) dvr[k] = ok[k] ? ldg_global<u32x4>(drow + (int64_t)chunk[k] * 16) : u32x4{0, 0, 0, 0};
    }
  };
  if (S > 0 && (int64_t)blockIdx.x < P.n_tokens) load_row(blockIdx.x);
  if constexpr (!MULTIQ) {
    // query and gain issued back to back, folded after both arrive
    ParamRaw<VEC> rq[V], rg[V];
#pragma unroll
    for (int k = 0; k < V; ++k) {
      if (!ok[k]) continue;
      load_param_raw<VEC>(P.query, chunk[k], P.param_bf16, rq[k]);
      if (P.gain != nullptr) load_param_raw<VEC>(P.gain, chunk[k], P.param_bf16, rg[k]);
    }
#pragma unroll
    for (int k = 0; k < V; ++k) {
      float t[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        if (!ok[k]) {
          t[e] = 0.f;
          continue;
        }
        const float qv = param_elem<VEC>(rq[k], e, P.param_bf16);
        if (P.gain != nullptr) {
          const float prod = qv * param_elem<VEC>(rg[k], e, P.param_bf16);
          t[e] = P.param_bf16 ? round_bf16(prod) : prod;
        } else {
          t[e] = qv;
        }
      }
      set_qw(k, t);
    }
  }

  int ph = 0;

  for (int64_t tok = blockIdx.x; tok < P.n_tokens; tok += gridDim.x) {
    if constexpr (S == 0) {
      // Softmax over an empty set is NaN everywhere (llama.py:642-644 with an
      // all-false mask; kernels/phase_1.py:78-101 with num_active == 0).
      const float nan = __builtin_nanf("");
      for (int q = 0; q < nq; ++q) {
        char* orow = reinterpret_cast<char*>(P.out) +
                     ((int64_t)q * P.out_qstride + tok * P.out_ld) * (P.out_bf16 ? 2 : 4);
#pragma unroll
        for (int k = 0; k < V; ++k) {
          if (!ok[k]) continue;
          if (P.out_bf16) {
            uint32_t h = pack_bf16(nan, nan);
            if constexpr (VEC == 8) stg<u32x4>(orow + (int64_t)chunk[k] * 16, u32x4{h, h, h, h});
            else stg<u32x2>(orow + (int64_t)chunk[k] * 8, u32x2{h, h});
          } else {
            const uint32_t f = __builtin_bit_cast(uint32_t, nan);
            u32x4 v = {f, f, f, f};
            if constexpr (VEC == 8) {
              stg<u32x4>(orow + (int64_t)chunk[k] * 32, v);
              stg<u32x4>(orow + (int64_t)chunk[k] * 32 + 16, v);
            } else {
              stg<u32x4>(orow + (int64_t)chunk[k] * 16, v);
            }
          }
        }
        if (tid == 0 && P.lse) P.lse[(int64_t)q * P.n_tokens + tok] = nan;
      }
      continue;
    } else {
      // ---- fused partial update: partial (+)= delta, written back ----
      if (P.mode != ATTNRES_MODE_PLAIN) {
#pragma unroll
        for (int k = 0; k < V; ++k) {
          if (!ok[k]) continue;
          const u32x4 dv = dvr[k];
          u32x4 nv = dv;
          if (P.mode == ATTNRES_MODE_ACCUM) {
            if constexpr (BF16) {
#pragma unroll
              for (int w = 0; w < 4; ++w)
                nv[w] = pack_bf16(bf_lo(x[S - 1][k][w]) + bf_lo(dv[w]), bf_hi(x[S - 1][k][w]) + bf_hi(dv[w]));
            } else {
#pragma unroll
              for (int w = 0; w < 4; ++w)
                nv[w] = as_u32(as_f32(x[S - 1][k][w]) + as_f32(dv[w]));
            }
          }
          x[S - 1][k] = nv;
        }
      }

      for (int q = 0; q < nq; ++q) {
        if constexpr (MULTIQ) fetch_qw(q);

        // ---- per-thread partial sums ----
        float part[NP];
#pragma unroll
        for (int j = NV; j < NP; ++j) part[j] = 0.f;
#pragma unroll
        for (int s = 0; s < S; ++s) {
          float ss = 0.f, dt = 0.f;
#pragma unroll
          for (int k = 0; k < V; ++k) {
            if constexpr (BF16) {
#pragma unroll
              for (int w = 0; w < 4; ++w) {
                ss = dot2_bf16(x[s][k][w], x[s][k][w], ss);
                if constexpr (QDOT2) {
                  dt = dot2_bf16(x[s][k][w], qwb[k][w], dt);
                } else {
                  dt = __builtin_fmaf(bf_lo(x[s][k][w]), qwf[k][2 * w], dt);
                  dt = __builtin_fmaf(bf_hi(x[s][k][w]), qwf[k][2 * w + 1], dt);
                }
              }
            } else {
#pragma unroll
              for (int e = 0; e < VEC; ++e) {
                const float v = C::elem(x[s][k], e);
                ss = __builtin_fmaf(v, v, ss);
                dt = __builtin_fmaf(v, qwf[k][e], dt);
              }
            }
          }
          part[s] = ss;
          part[S + s] = dt;
        }

        // ---- transposing wave reduction, one LDS exchange across the waves ----
        wave_reduce_to_lds<NP / 4>(part, red[ph][wave], lane);
        __syncthreads();

        // ---- softmax over depth, lane s per source (segments of SEG lanes) ----
        float t_ss = 0.f, t_dot = 0.f;
        if (slot) {
          for (int w = 0; w < nwaves; ++w) {
            t_ss += red[ph][w][ls];
            t_dot += red[ph][w][S + ls];
          }
        }
        ph ^= 1;
        const float inv = __builtin_amdgcn_rsqf(t_ss * P.inv_d + P.eps);
        const float logit = slot ? t_dot * inv : -__builtin_inff();
        const float m = seg_max<SEG>(logit);
        const float el = slot ? __expf(logit - m) : 0.f;
        const float sum = seg_sum<SEG>(el);
        const float wl = el * (1.0f / sum);
        if (wave == 0 && lane < S) {
          if (P.weights) P.weights[((int64_t)q * S + lane) * P.n_tokens + tok] = wl;
          if (P.logits) P.logits[((int64_t)q * P.n_tokens + tok) * S + lane] = logit;
          if (q == 0 && P.inv_rms) P.inv_rms[tok * S + lane] = inv;
          if (lane == 0 && P.lse) P.lse[(int64_t)q * P.n_tokens + tok] = m + __logf(sum);
        }
        float wgt[S];
#pragma unroll
        for (int s = 0; s < S; ++s)
          wgt[s] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), s));

        // ---- weighted sum of the raw sources, one output row ----
        // The empty asm makes the rows opaque here, so the compiler re-unpacks
        // bf16 pairs below instead of keeping the fp32 copies from the dot
        // phase alive (which doubles register use).
#pragma unroll
        for (int s = 0; s < S; ++s) {
#pragma unroll
          for (int k = 0; k < V; ++k) asm volatile("" : "+v"(x[s][k]));
        }
        char* orow = reinterpret_cast<char*>(P.out) +
                     ((int64_t)q * P.out_qstride + tok * P.out_ld) * (P.out_bf16 ? 2 : 4);
        const __amdgpu_buffer_rsrc_t orsrc = row_rsrc(orow, (uint32_t)(P.d * (P.out_bf16 ? 2 : 4)));
#pragma unroll
        for (int k = 0; k < V; ++k) {
          if (!ok[k]) continue;
          float acc[VEC];
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc[e] = wgt[0] * C::elem(x[0][k], e);
#pragma unroll
          for (int s = 1; s < S; ++s) {
#pragma unroll
            for (int e = 0; e < VEC; ++e) acc[e] = __builtin_fmaf(wgt[s], C::elem(x[s][k], e), acc[e]);
          }
          if (P.out_bf16) {
            if constexpr (VEC == 8) {
              st_row(orsrc, (uint32_t)chunk[k] * 16,
                     u32x4{pack_bf16(acc[0], acc[1]), pack_bf16(acc[2], acc[3]), pack_bf16(acc[4], acc[5]),
                           pack_bf16(acc[6], acc[7])});
            } else {
              st_row(orsrc, (uint32_t)chunk[k] * 8, u32x2{pack_bf16(acc[0], acc[1]), pack_bf16(acc[2], acc[3])});
            }
          } else {
#pragma unroll
            for (int h = 0; h < VEC / 4; ++h) {
              st_row(orsrc, ((uint32_t)chunk[k] * VEC + 4 * h) * 4,
                         u32x4{as_u32(acc[4 * h]), as_u32(acc[4 * h + 1]),
                               as_u32(acc[4 * h + 2]),
                               as_u32(acc[4 * h + 3])});
            }
          }
        }
      }
      // The updated partial row is written back (or to partial_out) after the
      // output row: a store issued before the dot products would be waited for
      // with the loads.
      if (P.mode != ATTNRES_MODE_PLAIN) {
        void* pdst = P.partial_out != nullptr ? P.partial_out : const_cast<void*>(P.src[S - 1]);
        char* prow = reinterpret_cast<char*>(pdst) + tok * row_bytes_ld;
        const __amdgpu_buffer_rsrc_t prsrc = row_rsrc(prow, (uint32_t)(P.d * C::BYTES));
#pragma unroll
        for (int k = 0; k < V; ++k) {
          if (ok[k]) st_row(prsrc, (uint32_t)chunk[k] * 16, x[S - 1][k]);
        }
      }
      if (tok + gridDim.x < P.n_tokens) load_row(tok + gridDim.x);
    }
  }
}

// ------------------------------------------------- batched-query body --
//
// Phase-1 batching for bf16 sources and bf16 parameters (the serving
// engine's case): Q >= 2 pseudo-queries over one set of sources.  One
// workgroup per token row, the S source chunks loaded once per row.  The Q
// folded queries are staged in LDS once per workgroup (packed bf16).  Per
// group of QG queries:
//  * sum(x^2) (once per row) and every x.qw with v_dot2_f32_bf16;
//  * the NV partial sums are reduced over the wave by a transposing tree:
//    v_permlane32_swap and v_permlane16_swap exchange half of the values
//    between lane halves (one instruction moves two registers' halves), so
//    each register carries four different values, one per 16-lane row, and
//    four DPP steps finish the row sums: ~2.5 instructions per value instead
//    of 6 for a full DPP reduction of each;
//  * one LDS exchange and one barrier; lane g*SEG + s then sums value (g, s)
//    over the waves and runs the QG depth softmaxes in parallel, SEG-lane
//    segments reduced with DPP (max, sum);
//  * mixing on the matrix cores (groups of a multiple of 4 queries): per
//    element of a lane, out[q] = sum_s w[q][s] x_s is column j of a 4x4x4
//    block product whose k runs over four sources: B is the lane's own
//    sources at that element (two v_perm_b32 per source pair and element
//    pair), A the weights of four queries, moved from the softmax lanes
//    with ds_bpermute and split into a bf16 hi and lo part (w = hi + lo to
//    2^-18 relative; each product and the sum are fp32), two MFMAs per
//    four sources.  Groups of 2 queries (S >= 13) mix on the VALU: the
//    weights move to scalar registers (v_readlane) and each source word is
//    unpacked once for all the group's output rows.

// Queries per group: one lane per (query, source) in the softmax (QG * SEG
// <= 64 lanes); groups of 8 up to S = 8 (at S = 6-8 they cost occupancy,
// 2 waves per SIMD instead of 3-4, and still measured 2-3% faster than
// groups of 4 with the mixing on the matrix cores).
#ifndef QG_OF
#define QG_OF(S) ((S) <= 8 ? 8 : (S) <= 12 ? 4 : 2)
#endif
#define ATTNRES_QG_MAX_NP 72  // partial sums of a group: 4 * ceil(S * (QG + 1) / 4), S = 8 with QG = 8

template <int S, int V>
__device__ __forceinline__ void route_qg_body(const attnres_route_params& P) {
  constexpr int VEC = 8;
  constexpr int QG = QG_OF(S);
  constexpr int SEG = S <= 8 ? 8 : 16;      // lanes per query in the softmax
  constexpr int NV = S * (QG + 1);          // sum(x^2) per source, then x.qw per (query, source)
  constexpr int H2 = (NV + 3) / 4;          // registers after the two swap rounds
  constexpr int NP = 4 * H2;                // NV padded to a multiple of 4
  static_assert(QG * SEG <= 64 && NP <= ATTNRES_QG_MAX_NP, "one lane per (query, source); reduction rows fit");
  __shared__ float red[2][ATTNRES_KMAX_WAVES][ATTNRES_QG_MAX_NP];
  extern __shared__ u32x4 qg_lds[];  // [query][chunk] packed folded queries

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int block = P.block;
  const int nwaves = (block + 63) >> 6;
  const int nq = P.num_queries;
  const int nchunk = P.nchunk;

  int chunk[V], qchunk[V];
#pragma unroll
  for (int k = 0; k < V; ++k) {
    chunk[k] = tid + k * block;
    qchunk[k] = chunk[k] < nchunk ? chunk[k] : nchunk - 1;  // rows past the end hold zeros
  }

  // ---- the batch's folded queries into LDS, once per workgroup ----
  for (int i = tid; i < nq * nchunk; i += block) {
    const int q = i / nchunk, c = i - q * nchunk;
    float t[VEC];
    load_qw<VEC>(P, q, c, t);
    qg_lds[i] = u32x4{pack_bf16(t[0], t[1]), pack_bf16(t[2], t[3]), pack_bf16(t[4], t[5]), pack_bf16(t[6], t[7])};
  }

  // Source rows through buffer resources: a chunk past the row end reads 0.
  const int64_t row_bytes_ld = P.src_ld * 2;
  u32x4 x[S][V];
  auto load_row = [&](int64_t t) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      char* row = reinterpret_cast<char*>(const_cast<void*>(P.src[s])) + t * row_bytes_ld;
      const __amdgpu_buffer_rsrc_t rs = row_rsrc(row, (uint32_t)(P.d * 2));
#pragma unroll
      for (int k = 0; k < V; ++k) x[s][k] = ld_row(rs, (uint32_t)chunk[k] * 16);
    }
  };
  if ((int64_t)blockIdx.x < P.n_tokens) load_row(blockIdx.x);

  // The softmax lane of this thread: query g of the group, source s.
  const int sg = lane / SEG, ss = lane % SEG;
  const bool slot = ss < S && sg < QG;
  __syncthreads();

  int ph = 0;
  for (int64_t tok = blockIdx.x; tok < P.n_tokens; tok += gridDim.x) {
    // sum(x^2) partials, once per row; every group reduces them again (the
    // same values), which costs less than selecting them out of later groups
    float ssp[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
      ssp[s] = 0.f;
#pragma unroll
      for (int k = 0; k < V; ++k) {
#pragma unroll
        for (int w = 0; w < 4; ++w) ssp[s] = dot2_bf16(x[s][k][w], x[s][k][w], ssp[s]);
      }
    }
    for (int q0 = 0; q0 < nq; q0 += QG) {
      const int ng = nq - q0 < QG ? nq - q0 : QG;

      // ---- the group's x.qw, packed dot products ----
      float part[NP];
#pragma unroll
      for (int j = 0; j < NP; ++j) part[j] = j < S ? ssp[j] : 0.f;
#pragma unroll
      for (int k = 0; k < V; ++k) {
        u32x4 qv[QG];
#pragma unroll
        for (int g = 0; g < QG; ++g) {
          const int q = q0 + g < nq ? q0 + g : nq - 1;  // a repeated query past the batch: weights unused
          qv[g] = qg_lds[q * nchunk + qchunk[k]];
        }
#pragma unroll
        for (int s = 0; s < S; ++s) {
#pragma unroll
          for (int w = 0; w < 4; ++w) {
#pragma unroll
            for (int g = 0; g < QG; ++g) part[S + g * S + s] = dot2_bf16(x[s][k][w], qv[g][w], part[S + g * S + s]);
          }
        }
      }

      // ---- transposing wave reduction, one LDS exchange ----
      wave_reduce_to_lds<H2>(part, red[ph][wave], lane);
      __syncthreads();

      // ---- totals over the waves and the softmaxes, one lane per (query, source) ----
      const int vi = S + sg * S + ss;
      float dot = 0.f, sq = 0.f;
      if (slot) {
        for (int w = 0; w < nwaves; ++w) {
          dot += red[ph][w][vi];
          sq += red[ph][w][ss];
        }
      }
      ph ^= 1;
      const float inv = __builtin_amdgcn_rsqf(sq * P.inv_d + P.eps);
      const float logit = slot ? dot * inv : -__builtin_inff();
      const float m = seg_max<SEG>(logit);
      const float e = slot ? __expf(logit - m) : 0.f;
      const float sum = seg_sum<SEG>(e);
      const float wl = e * (1.0f / sum);
      if (wave == 0 && slot && sg < ng) {
        const int q = q0 + sg;
        if (P.weights) P.weights[((int64_t)q * S + ss) * P.n_tokens + tok] = wl;
        if (P.logits) P.logits[((int64_t)q * P.n_tokens + tok) * S + ss] = logit;
        if (P.lse && ss == 0) P.lse[(int64_t)q * P.n_tokens + tok] = m + __logf(sum);
        if (P.inv_rms && q0 == 0 && sg == 0) P.inv_rms[tok * S + ss] = inv;
      }
      if constexpr (QG % 4 == 0) {
        // ---- mixing on the matrix cores ----
        constexpr int NG4 = QG / 4, KS = (S + 3) / 4;
        // A operands: lane 4b+i takes the weights of query q0 + 4*g4 + i over
        // sources 4*ks .. 4*ks+3 (zero past S) from the softmax lanes
        const int ai = lane & 3;
        u32x2 ahi[NG4][KS], alo[NG4][KS];
#pragma unroll
        for (int g4 = 0; g4 < NG4; ++g4) {
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) {
            float wv[4];
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
              const int sidx = 4 * ks + kk;
              wv[kk] = sidx < S ? __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(
                                                                ((4 * g4 + ai) * SEG + sidx) * 4,
                                                                __builtin_bit_cast(int, wl)))
                                : 0.f;
            }
            const uint32_t h01 = pack_bf16(wv[0], wv[1]), h23 = pack_bf16(wv[2], wv[3]);
            ahi[g4][ks] = u32x2{h01, h23};
            alo[g4][ks] = u32x2{pack_bf16(wv[0] - bf_lo(h01), wv[1] - bf_hi(h01)),
                                pack_bf16(wv[2] - bf_lo(h23), wv[3] - bf_hi(h23))};
          }
        }
#pragma unroll
        for (int sidx = 0; sidx < S; ++sidx) {
#pragma unroll
          for (int k = 0; k < V; ++k) asm volatile("" : "+v"(x[sidx][k]));
        }
#pragma unroll
        for (int k = 0; k < V; ++k) {
          // acc[h][g4][i]: out[q0 + 4*g4 + i] at element h of this lane's chunk
          f32x4 acc[8][NG4];
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            // B operands of elements 2w (low halves) and 2w+1 (high halves)
            u32x2 blo[KS], bhi[KS];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
              for (int p = 0; p < 2; ++p) {
                const int s0 = 4 * ks + 2 * p, s1 = s0 + 1;
                const uint32_t a = s0 < S ? x[s0][k][w] : 0u;
                const uint32_t b = s1 < S ? x[s1][k][w] : 0u;
                blo[ks][p] = __builtin_amdgcn_perm(b, a, 0x05040100u);
                bhi[ks][p] = __builtin_amdgcn_perm(b, a, 0x07060302u);
              }
            }
#pragma unroll
            for (int g4 = 0; g4 < NG4; ++g4) {
              f32x4 cl = {0.f, 0.f, 0.f, 0.f}, ch = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
              for (int ks = 0; ks < KS; ++ks) {
                cl = mfma_4x4x4(ahi[g4][ks], blo[ks], cl);
                ch = mfma_4x4x4(ahi[g4][ks], bhi[ks], ch);
                cl = mfma_4x4x4(alo[g4][ks], blo[ks], cl);
                ch = mfma_4x4x4(alo[g4][ks], bhi[ks], ch);
              }
              acc[2 * w][g4] = cl;
              acc[2 * w + 1][g4] = ch;
            }
          }
          // chunks past the row end fall outside the buffer range: the store is dropped
#pragma unroll
          for (int g4 = 0; g4 < NG4; ++g4) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int g = 4 * g4 + i;
              if (g >= ng) continue;
              char* orow = reinterpret_cast<char*>(P.out) + ((int64_t)(q0 + g) * P.out_qstride + tok * P.out_ld) * 2;
              st_row(row_rsrc(orow, (uint32_t)(P.d * 2)), (uint32_t)chunk[k] * 16,
                     u32x4{pack_bf16(acc[0][g4][i], acc[1][g4][i]), pack_bf16(acc[2][g4][i], acc[3][g4][i]),
                           pack_bf16(acc[4][g4][i], acc[5][g4][i]), pack_bf16(acc[6][g4][i], acc[7][g4][i])});
            }
          }
        }
      } else {
        float wgt[QG][S];
#pragma unroll
        for (int g = 0; g < QG; ++g) {
#pragma unroll
          for (int s = 0; s < S; ++s)
            wgt[g][s] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), g * SEG + s));
        }

        // ---- mixing: each source word unpacked once for all the group's rows ----
#pragma unroll
        for (int s = 0; s < S; ++s) {
#pragma unroll
          for (int k = 0; k < V; ++k) asm volatile("" : "+v"(x[s][k]));
        }
#pragma unroll
        for (int k = 0; k < V; ++k) {
          uint32_t ow[QG][4];
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            float xl[S], xh[S];
#pragma unroll
            for (int s = 0; s < S; ++s) {
              xl[s] = bf_lo(x[s][k][w]);
              xh[s] = bf_hi(x[s][k][w]);
            }
#pragma unroll
            for (int g = 0; g < QG; ++g) {
              float lo = wgt[g][0] * xl[0], hi = wgt[g][0] * xh[0];
#pragma unroll
              for (int s = 1; s < S; ++s) {
                lo = __builtin_fmaf(wgt[g][s], xl[s], lo);
                hi = __builtin_fmaf(wgt[g][s], xh[s], hi);
              }
              ow[g][w] = pack_bf16(lo, hi);
            }
          }
          // chunks past the row end fall outside the buffer range: the store is dropped
#pragma unroll
          for (int g = 0; g < QG; ++g) {
            if (g >= ng) continue;
            char* orow = reinterpret_cast<char*>(P.out) + ((int64_t)(q0 + g) * P.out_qstride + tok * P.out_ld) * 2;
            st_row(row_rsrc(orow, (uint32_t)(P.d * 2)), (uint32_t)chunk[k] * 16,
                   u32x4{ow[g][0], ow[g][1], ow[g][2], ow[g][3]});
          }
        }
      }
    }
    if (tok + gridDim.x < P.n_tokens) load_row(tok + gridDim.x);
  }
}

// ------------------------------------------------------------ merge body --

// One VEC-element chunk of a bf16 (GBF) or fp32 row, packed as loaded.
template <int VEC, bool GBF>
struct PackedChunk {
  static constexpr int WORDS = VEC * (GBF ? 2 : 4) / 4;
  uint32_t w[WORDS];
  __device__ __forceinline__ void load(const char* row, int chunk) {
    const char* p = row + (int64_t)chunk * (WORDS * 4);
    if constexpr (WORDS == 2) {
      const u32x2 t = ldg_global<u32x2>(p);
      w[0] = t[0];
      w[1] = t[1];
    } else {
#pragma unroll
      for (int h = 0; h < WORDS / 4; ++h) {
        const u32x4 t = ldg_global<u32x4>(p + h * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) w[4 * h + i] = t[i];
      }
    }
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < WORDS; ++i) w[i] = 0u;
  }
  __device__ __forceinline__ float elem(int e) const {
    if constexpr (GBF) return (e & 1) ? bf_hi(w[e >> 1]) : bf_lo(w[e >> 1]);
    else return as_f32(w[e]);
  }
};


// Phase-2 merge of the intra-block partial into the phase-1 inter-block
// result (kernels/phase_2.py:40-57 semantics): one token row per workgroup.
template <int V, bool PBF16, bool IBF16>
__device__ __forceinline__ void merge_body(const attnres_merge_params& P) {
  using C = Chunk<PBF16>;
  constexpr int VEC = C::VEC;
  using IC = PackedChunk<VEC, IBF16>;
  __shared__ float red[2][ATTNRES_KMAX_WAVES][4];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int block = P.block;
  const int nwaves = (block + 63) >> 6;

  int chunk[V];
  bool ok[V];
#pragma unroll
  for (int k = 0; k < V; ++k) {
    chunk[k] = tid + k * block;
    ok[k] = chunk[k] < P.nchunk;
  }
  // The row (partial and inter, packed) is requested before the query, so a
  // workgroup that owns one row waits for memory once.
  u32x4 p[V];
  IC ic[V];
  auto load_row = [&](int64_t t) {
    const char* prow = reinterpret_cast<const char*>(P.partial) + t * P.partial_ld * C::BYTES;
    const char* irow = reinterpret_cast<const char*>(P.inter) + t * P.inter_ld * (IBF16 ? 2 : 4);
#pragma unroll
    for (int k = 0; k < V; ++k) {
      if (ok[k]) {
        p[k] = ldg_global<u32x4>(prow + (int64_t)chunk[k] * 16);
        ic[k].load(irow, chunk[k]);
      } else {
        p[k] = u32x4{0, 0, 0, 0};
        ic[k].zero();
      }
    }
  };
  if ((int64_t)blockIdx.x < P.n_tokens) load_row(blockIdx.x);
  float qw[V][VEC];
#pragma unroll
  for (int k = 0; k < V; ++k) {
    if (ok[k]) {
      load_param<VEC>(P.query, (int64_t)chunk[k] * VEC, P.param_bf16, qw[k]);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) qw[k][e] = 0.f;
    }
  }

  int ph = 0;
  for (int64_t tok = blockIdx.x; tok < P.n_tokens; tok += gridDim.x) {
    float ss = 0.f, dt = 0.f;
#pragma unroll
    for (int k = 0; k < V; ++k) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float v = C::elem(p[k], e);
        ss = __builtin_fmaf(v, v, ss);
        dt = __builtin_fmaf(v, qw[k][e], dt);
      }
    }
    ss = wave_sum_to_lane63(ss);
    dt = wave_sum_to_lane63(dt);
    if (lane == 63) {
      red[ph][wave][0] = ss;
      red[ph][wave][1] = dt;
    }
    __syncthreads();
    float tss = 0.f, tdt = 0.f;
    for (int w = 0; w < nwaves; ++w) {
      tss += red[ph][w][0];
      tdt += red[ph][w][1];
    }
    ph ^= 1;
    const float inv = __builtin_amdgcn_rsqf(tss * P.inv_d + P.eps);
    const float logit = tdt * inv;
    const float pi = 1.0f / (1.0f + __expf(-(logit - P.inter_lse[tok])));
    if (tid == 0) {
      if (P.logit) P.logit[tok] = logit;
      if (P.inv_rms) P.inv_rms[tok] = inv;
    }

    char* orow = reinterpret_cast<char*>(P.out) + tok * P.out_ld * (IBF16 ? 2 : 4);
    const __amdgpu_buffer_rsrc_t orsrc = row_rsrc(orow, (uint32_t)(P.d * (IBF16 ? 2 : 4)));
#pragma unroll
    for (int k = 0; k < V; ++k) {
      if (!ok[k]) continue;
      float o[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float iv = ic[k].elem(e);
        o[e] = __builtin_fmaf(pi, C::elem(p[k], e) - iv, iv);
      }
      if constexpr (IBF16) {
        if constexpr (VEC == 8) {
          st_row(orsrc, (uint32_t)chunk[k] * 16,
                 u32x4{pack_bf16(o[0], o[1]), pack_bf16(o[2], o[3]), pack_bf16(o[4], o[5]), pack_bf16(o[6], o[7])});
        } else {
          st_row(orsrc, (uint32_t)chunk[k] * 8, u32x2{pack_bf16(o[0], o[1]), pack_bf16(o[2], o[3])});
        }
      } else {
#pragma unroll
        for (int h = 0; h < VEC / 4; ++h) {
          st_row(orsrc, ((uint32_t)chunk[k] * VEC + 4 * h) * 4,
                     u32x4{as_u32(o[4 * h]), as_u32(o[4 * h + 1]),
                           as_u32(o[4 * h + 2]), as_u32(o[4 * h + 3])});
        }
      }
    }
    if (tok + gridDim.x < P.n_tokens) load_row(tok + gridDim.x);
  }
}

// Phase-2 merge, one wave per token row (bf16 partial, inter and output rows
// of NCH KiB): lane l holds the 16-byte chunks l, l+64, ... of a row.  The
// wave's rows stream through a two-slot register pipeline one row per slot,
// as the routing kernel's sources do: slot A takes token t's partial row,
// slot B its inter row, and each load is requested before the previous row
// is processed.  From the partial row: sum(p^2) and p.q per lane, one DPP
// wave reduction each, pi = sigmoid((p.q) r - lse), r = rsqrt(mean(p^2) +
// eps); the partial row is kept while the inter row arrives, then
//   out = inter + pi (p - inter)
// and one store of the row.  The query sits in LDS (bf16 pairs for the
// v_dot2 path when the parameter is bf16, else fp32), read once per
// workgroup.  Same arithmetic as merge_body; only the order of the row sums
// differs.
template <int NCH, bool QDOT2>
__device__ __forceinline__ void merge_stream_body(const attnres_merge_params& P) {
  constexpr int QF = QDOT2 ? 1 : NCH * 64 * 8;
  constexpr int QB = QDOT2 ? NCH * 64 : 1;
  __shared__ u32x4 qw_b[QB];
  __shared__ float qw_f[QF];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  for (int i = tid; i < NCH * 64; i += blockDim.x) {
    float t[8];
    load_param<8>(P.query, (int64_t)i * 8, P.param_bf16, t);
    if constexpr (QDOT2) {
      qw_b[i] = u32x4{pack_bf16(t[0], t[1]), pack_bf16(t[2], t[3]), pack_bf16(t[4], t[5]), pack_bf16(t[6], t[7])};
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) qw_f[i * 8 + e] = t[e];
    }
  }
  __syncthreads();

  // 32-bit wave-uniform row counters (the host checks n_tokens < 2^31)
  const uint32_t n_tok = (uint32_t)P.n_tokens;
  const uint32_t wpb = __builtin_amdgcn_readfirstlane((uint32_t)P.block >> 6);
  const uint32_t nw = gridDim.x * wpb;
  uint32_t tok = blockIdx.x * wpb + wave;
  if (tok >= n_tok) return;  // no barrier follows
  // wave-uniform (the division is expanded on the VALU): a loop bound in a
  // VGPR would make the row loop divergent
  const uint32_t rows = __builtin_amdgcn_readfirstlane((n_tok - tok - 1) / nw + 1);
  const uint64_t p0 = reinterpret_cast<uint64_t>(P.partial), i0 = reinterpret_cast<uint64_t>(P.inter);
  const uint64_t o0 = reinterpret_cast<uint64_t>(P.out);
  const uint64_t p_ld = (uint64_t)P.partial_ld * 2, i_ld = (uint64_t)P.inter_ld * 2, o_ld = (uint64_t)P.out_ld * 2;

  // rows are read once: global loads with the non-temporal hint, as the
  // routing kernels' source rows
  auto load_row = [&](u32x4(&buf)[NCH], uint64_t base, uint64_t ld, uint32_t t) {
    t = __builtin_amdgcn_readfirstlane(t);
    const char* row = uniform_ptr(base + (uint64_t)t * ld);
#pragma unroll
    for (int c = 0; c < NCH; ++c) buf[c] = ldg_global<u32x4>(row + (uint32_t)(c * 1024 + lane * 16));
    __builtin_amdgcn_sched_barrier(0);
  };
  u32x4 pa[NCH], ib[NCH], ph[NCH];
  // The lse of a token is requested with its partial row, a row ahead of its
  // use: a scalar load counts against the same wait counter as the LDS reads
  // of the query, so one requested just before use would stall every row.
  load_row(pa, p0, p_ld, tok);
  float lse_next = P.inter_lse[tok];
  for (uint32_t i = 0; i < rows; ++i) {
    const uint32_t tn = i + 1 < rows ? tok + nw : tok;  // past the last row: re-read a valid row
    const float lse = lse_next;
    load_row(ib, i0, i_ld, tok);
    // ---- the partial row: sum(p^2), p.q, pi ----
    asm volatile("; attnres merge stream partial");
    float ss0 = 0.f, ss1 = 0.f, dt0 = 0.f, dt1 = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if constexpr (QDOT2) {
        const u32x4 q = qw_b[c * 64 + lane];
        ss0 = dot2_bf16(pa[c][0], pa[c][0], ss0);
        dt0 = dot2_bf16(pa[c][0], q[0], dt0);
        ss1 = dot2_bf16(pa[c][1], pa[c][1], ss1);
        dt1 = dot2_bf16(pa[c][1], q[1], dt1);
        ss0 = dot2_bf16(pa[c][2], pa[c][2], ss0);
        dt0 = dot2_bf16(pa[c][2], q[2], dt0);
        ss1 = dot2_bf16(pa[c][3], pa[c][3], ss1);
        dt1 = dot2_bf16(pa[c][3], q[3], dt1);
      } else {
        const float* q = &qw_f[(c * 64 + lane) * 8];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float a = bf_lo(pa[c][w]), b = bf_hi(pa[c][w]);
          ss0 = __builtin_fmaf(a, a, ss0);
          dt0 = __builtin_fmaf(a, q[2 * w], dt0);
          ss1 = __builtin_fmaf(b, b, ss1);
          dt1 = __builtin_fmaf(b, q[2 * w + 1], dt1);
        }
      }
    }
    float ss = wave_sum_to_lane63(ss0 + ss1);
    float dt = wave_sum_to_lane63(dt0 + dt1);
    ss = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ss), 63));
    dt = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, dt), 63));
    const float inv = __builtin_amdgcn_rsqf(ss * P.inv_d + P.eps);
    const float logit = dt * inv;
    const float pi = 1.0f / (1.0f + __expf(-(logit - lse)));
    if (lane == 0) {
      if (P.logit) P.logit[tok] = logit;
      if (P.inv_rms) P.inv_rms[tok] = inv;
    }
    // keep the partial row; its slot takes the next token's partial row
#pragma unroll
    for (int c = 0; c < NCH; ++c) ph[c] = pa[c];
    load_row(pa, p0, p_ld, tn);
    lse_next = P.inter_lse[tn];
    // ---- the inter row: out = inter + pi (p - inter) ----
    asm volatile("; attnres merge stream inter");
    const __amdgpu_buffer_rsrc_t orr = row_rsrc(const_cast<char*>(uniform_ptr(o0 + (uint64_t)tok * o_ld)), NCH * 1024);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      u32x4 o;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float il = bf_lo(ib[c][w]), ih = bf_hi(ib[c][w]);
        o[w] = pack_bf16(__builtin_fmaf(pi, bf_lo(ph[c][w]) - il, il), __builtin_fmaf(pi, bf_hi(ph[c][w]) - ih, ih));
      }
      st_row(orr, (uint32_t)(c * 1024 + lane * 16), o);
    }
    tok = __builtin_amdgcn_readfirstlane(tn);
  }
}


// ------------------------------------------------------ stream body --
//
// Prefill kernel: one wave64 owns one token row at a time, and the S source
// rows stream through a two-deep register pipeline (slots A and B): the load
// of the next (token, source) item is issued as soon as the current one has
// arrived and before it is processed, across token boundaries, so every wave
// keeps exactly one row of HBM reads in flight.  Lane l holds the 16-byte chunks l, l+64, ... (NCH chunks of a
// row of NCH KiB), so each wave-wide load covers 1 KiB contiguous.
//
// Per source: sum(x^2) and x.qw over the lane's chunks, one DPP wave
// reduction each (no LDS, no barrier), then an online depth softmax with
// wave-uniform state (m, l):
//   first source      m = logit, l = 1,               acc = x
//   new maximum       c = exp(m - logit), l = l*c+1,  acc = acc*c + x
//   otherwise         p = exp(logit - m), l += p,     acc = acc + p*x
// so the rescale and the accumulate are one FMA per element.  The output row
// is acc / l; lse = m + log(l).  Lane s keeps logit_s and inv_rms_s for the
// optional weight / aux outputs.  qw sits in LDS, loaded once per workgroup.
//
// FUSED: the last slot is the partial block, updated in-kernel from `delta`
// (MODE_ACCUM: partial + delta, MODE_SET: delta) and written back; the delta
// row is prefetched with the partial row.

#define ATTNRES_STREAM_WAVES 4

// TBL: sources addressed through the kernel-argument pointer table (any
// pointers) instead of base + s * stride (equally spaced: stacked buffers,
// arenas).
template <int NCH, bool BF16, bool QDOT2, bool FUSED, bool OUTBF, bool TBL>
__device__ __forceinline__ void stream_body(const attnres_route_params& P) {
  const int S = P.num_sources;
  using C = Chunk<BF16>;
  constexpr int VEC = C::VEC;
  constexpr int QF = QDOT2 ? 1 : NCH * 64 * VEC;
  constexpr int QB = QDOT2 ? NCH * 64 : 1;
  __shared__ u32x4 qw_b[QB];
  __shared__ float qw_f[QF];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar loop control

  // ---- folded query into LDS, once per workgroup ----
  for (int i = tid; i < NCH * 64; i += blockDim.x) {
    float t[VEC];
    load_qw<VEC>(P, 0, i, t);
    if constexpr (QDOT2) {
      u32x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = pack_bf16(t[2 * e], t[2 * e + 1]);
      qw_b[i] = v;
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) qw_f[i * VEC + e] = t[e];
    }
  }
  __syncthreads();

  // Item counters are 32-bit and wave-uniform so all loop control and address
  // arithmetic stays in SGPRs (gfx9 has no scalar 64-bit signed compare).
  const uint32_t n_tok = (uint32_t)P.n_tokens;
  // waves per workgroup: up to ATTNRES_STREAM_WAVES, chosen at launch (P.block)
  const uint32_t wpb = __builtin_amdgcn_readfirstlane((uint32_t)P.block >> 6);
  const uint32_t nw = gridDim.x * wpb;
  uint32_t tok = blockIdx.x * wpb + wave;
  if (tok >= n_tok) return;  // no barrier follows

  const uint64_t row_bytes = (uint64_t)P.src_ld * C::BYTES;
  const uint64_t delta_row_bytes = (uint64_t)P.delta_ld * C::BYTES;
  const int mode = FUSED ? P.mode : ATTNRES_MODE_PLAIN;
  const uint64_t src0 = reinterpret_cast<uint64_t>(P.src[0]);
  const uint64_t src_stride = (uint64_t)P.src_stride;
  // Sources that are not equally spaced are addressed through the pointer
  // table of the kernel arguments, read with a scalar load at the
  // wave-uniform source index (indexing the by-value parameter struct would
  // copy it to scratch).
  typedef const __attribute__((address_space(4))) uint64_t kptr_u64;
  kptr_u64* src_tbl = (kptr_u64*)((const __attribute__((address_space(4))) char*)__builtin_amdgcn_kernarg_segment_ptr() +
                                   offsetof(attnres_route_params, src));
  const uint64_t delta0 = reinterpret_cast<uint64_t>(P.delta);

  u32x4 bufA[NCH], bufB[NCH];
  // Fused accumulate mode: the delta row of the token's partial source.  One
  // buffer serves both pipeline slots: with S >= 2 (the host sends S == 1
  // accumulate calls to the workgroup kernel) the two items in flight are
  // never both a token's last source, and the delta is consumed by the item
  // that loaded it before the next partial item is loaded.
  u32x4 dX[FUSED ? NCH : 1];

  // Sources are equally spaced (the host checks): source s of row t is at
  // src0 + s*src_stride + t*row_bytes, pure scalar arithmetic.
  // z: an arrival_zero() added to the lane offsets (0 for the first item).
  auto load_item = [&](u32x4(&buf)[NCH], u32x4(&dbuf)[FUSED ? NCH : 1], uint32_t t, uint32_t s, uint32_t z) {
    t = __builtin_amdgcn_readfirstlane(t);
    s = __builtin_amdgcn_readfirstlane(s);
    const bool from_delta = FUSED && s == (uint32_t)(S - 1) && mode == ATTNRES_MODE_SET;
    uint64_t base;
    if (from_delta) {
      base = delta0;
    } else if constexpr (TBL) {
      base = src_tbl[s];
    } else {
      base = src0 + (uint64_t)s * src_stride;
    }
    const char* row = uniform_ptr(base + (uint64_t)t * (from_delta ? delta_row_bytes : row_bytes));
#if ATTNRES_LOAD_CPOL >= 0
    const __amdgpu_buffer_rsrc_t rr = row_rsrc(const_cast<char*>(row), (uint32_t)(NCH * 1024));
#pragma unroll
    for (int c = 0; c < NCH; ++c) buf[c] = ld_row(rr, (uint32_t)(c * 1024 + lane * 16) + z);
#else
#pragma unroll
    for (int c = 0; c < NCH; ++c) buf[c] = ldg_global<u32x4>(row + ((uint32_t)(c * 1024 + lane * 16) + z));
#endif
    if constexpr (FUSED) {
      if (s == (uint32_t)(S - 1) && mode == ATTNRES_MODE_ACCUM) {
        const char* drow = uniform_ptr(delta0 + (uint64_t)t * delta_row_bytes);
#pragma unroll
        for (int c = 0; c < NCH; ++c) dbuf[c] = ldg_global<u32x4>(drow + (uint32_t)(c * 1024 + lane * 16));
      }
    }
    // keep the prefetch ahead of the work on the current row
    __builtin_amdgcn_sched_barrier(0);
  };

  float acc[NCH][VEC];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[c][e] = 0.f;
  }
  float m = -__builtin_inff(), l = 0.f;
  float my_logit = 0.f, my_inv = 0.f;  // lane s: logit and inv_rms of source s

  // ---- output rows ----
  // Store addresses: a wave-uniform row base (SGPRs) plus a 32-bit lane offset.
  constexpr int OES = OUTBF ? 2 : 4;                       // output element bytes
  constexpr int OPC = OUTBF ? 1 : VEC / 4;                 // pieces per lane and chunk
  constexpr int OPB = (OUTBF && VEC == 4) ? 8 : 16;        // bytes per piece
  auto out_rsrc = [&](uint32_t tt) {
    char* orow = const_cast<char*>(
        uniform_ptr(reinterpret_cast<uint64_t>(P.out) + (uint64_t)tt * (uint64_t)(P.out_ld * OES)));
    return row_rsrc(orow, (uint32_t)(P.d * OES));
  };
  // Byte offset of this lane's first output element, made opaque so the
  // per-chunk offsets are recomputed where used (mostly as immediate offsets)
  // rather than hoisted out of the loop and kept live in registers.
  auto lane_out_offset = [&]() {
    uint32_t lane_ob = (uint32_t)lane * (uint32_t)(VEC * OES);
    asm volatile("" : "+v"(lane_ob));
    return lane_ob;
  };
  // Finished rows can be staged in dynamic LDS (P.out_batch rows per wave,
  // plus REG_ROWS held in registers, below) and stored in batches: the
  // output stores then reach memory in bursts between long stretches of
  // pure reads, which this HBM serves far better than one row interleaved
  // after every S source rows (a store-only variant of the access pattern:
  // 78.5% -> 90.9% of peak at S = 8, batches of 8).  The staged layout is
  // [row][chunk][piece][lane] (consecutive lanes 8 or 16 bytes apart: no
  // bank conflicts); a wave reads back only what its own lanes wrote, so no
  // barrier is needed.  The fused variants store each row at once (their
  // partial write-back is a second write stream; staging measured slower
  // there) and carry no staging code.
  const uint32_t batch = (uint32_t)P.out_batch;
  // the arena's fused block steps (the partial written back in place) store
  // non-temporally; a fused step writing its partial to a new buffer does not
  const bool nt_st = FUSED && P.partial_out == nullptr;
  extern __shared__ u32x4 stream_stage[];
  constexpr uint32_t STAGE_ROW = NCH * OPC * 64 * OPB;     // bytes of one staged row
  auto stage_row = [&](uint32_t b) {
    return reinterpret_cast<char*>(stream_stage) + ((uint32_t)wave * batch + b) * STAGE_ROW;
  };
  // Past the LDS slots a wave holds REG_ROWS more finished rows in registers
  // (one wave per SIMD leaves the register file for it), so a batch is
  // P.out_batch + REG_ROWS rows: 8 and 10 row batches measured 1-1.5 points
  // of peak faster than the 6 the LDS holds at four waves (S = 4..8).
  constexpr int REG_ROWS = FUSED ? 1 : (NCH <= 6 ? 4 : 2);
  u32x4 held[REG_ROWS][NCH][OPC];
  const uint32_t full_batch = (!FUSED && batch > 1) ? batch + REG_ROWS : batch;
  uint32_t nheld = 0, t_first = 0;
  auto flush_staged = [&]() {
#pragma unroll
    for (int r = 0; r < REG_ROWS; ++r) {
      if (batch + (uint32_t)r < nheld) {
        const __amdgpu_buffer_rsrc_t orsrc = out_rsrc(t_first + (batch + r) * nw);
        const uint32_t lane_ob = lane_out_offset();
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
#pragma unroll
          for (int h = 0; h < OPC; ++h) {
            const uint32_t off = lane_ob + (uint32_t)(c * 64 * VEC * OES + 16 * h);
            if constexpr (OPB == 16) st_row(orsrc, off, held[r][c][h]);
            else st_row(orsrc, off, u32x2{held[r][c][h][0], held[r][c][h][1]});
          }
        }
      }
    }
    const uint32_t in_lds = nheld < batch ? nheld : batch;
    for (uint32_t b = 0; b < in_lds; ++b) {
      const __amdgpu_buffer_rsrc_t orsrc = out_rsrc(t_first + b * nw);
      const uint32_t lane_ob = lane_out_offset();
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
#pragma unroll
        for (int h = 0; h < OPC; ++h) {
          const char* sp = stage_row(b) + ((c * OPC + h) * 64 + lane) * OPB;
          const uint32_t off = lane_ob + (uint32_t)(c * 64 * VEC * OES + 16 * h);
          if constexpr (OPB == 16) st_row(orsrc, off, *reinterpret_cast<const u32x4*>(sp));
          else st_row(orsrc, off, *reinterpret_cast<const u32x2*>(sp));
        }
      }
    }
  };

  auto process = [&](u32x4(&x)[NCH], u32x4(&dbuf)[FUSED ? NCH : 1], uint32_t t, uint32_t s, auto slot) {
    // A distinct marker per pipeline slot keeps the compiler from merging the
    // two unrolled halves into one body (which would copy the row buffers
    // through phis and wait for the prefetch before using the current row).
    if constexpr (decltype(slot)::value == 0) {
      asm volatile("; attnres stream slot A");
    } else {
      asm volatile("; attnres stream slot B");
    }
    if constexpr (FUSED) {
      const bool wb = s == (uint32_t)(S - 1) && mode != ATTNRES_MODE_PLAIN;
      if (wb) {
        if (mode == ATTNRES_MODE_ACCUM) {
#pragma unroll
          for (int c = 0; c < NCH; ++c) {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
              if constexpr (BF16) {
                x[c][w] = pack_bf16(bf_lo(x[c][w]) + bf_lo(dbuf[c][w]), bf_hi(x[c][w]) + bf_hi(dbuf[c][w]));
              } else {
                x[c][w] = as_u32(as_f32(x[c][w]) + as_f32(dbuf[c][w]));
              }
            }
          }
        }
        // the updated partial row is written back, or to partial_out (in a
        // branch: an unconditional write-back through an empty resource made
        // these kernels spill)
        const uint64_t pout = reinterpret_cast<uint64_t>(P.partial_out);
        const uint64_t pbase = pout != 0 ? pout : TBL ? src_tbl[S - 1] : src0 + (uint64_t)(S - 1) * src_stride;
        char* prow = const_cast<char*>(uniform_ptr(pbase + (uint64_t)t * row_bytes));
        const __amdgpu_buffer_rsrc_t prsrc = row_rsrc(prow, (uint32_t)(NCH * 1024));
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
          if (nt_st) st_row_nt(prsrc, (uint32_t)(c * 1024 + lane * 16), x[c]);
          else st_row(prsrc, (uint32_t)(c * 1024 + lane * 16), x[c]);
        }
      }
    }

    // ---- sum(x^2) and x.qw over this lane's chunks (two chains each) ----
    float ss0 = 0.f, ss1 = 0.f, dt0 = 0.f, dt1 = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if constexpr (QDOT2) {
        const u32x4 q = qw_b[c * 64 + lane];
        ss0 = dot2_bf16(x[c][0], x[c][0], ss0);
        dt0 = dot2_bf16(x[c][0], q[0], dt0);
        ss1 = dot2_bf16(x[c][1], x[c][1], ss1);
        dt1 = dot2_bf16(x[c][1], q[1], dt1);
        ss0 = dot2_bf16(x[c][2], x[c][2], ss0);
        dt0 = dot2_bf16(x[c][2], q[2], dt0);
        ss1 = dot2_bf16(x[c][3], x[c][3], ss1);
        dt1 = dot2_bf16(x[c][3], q[3], dt1);
      } else {
        const float* q = &qw_f[(c * 64 + lane) * VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float v = C::elem(x[c], e);
          if (e & 1) {
            ss1 = __builtin_fmaf(v, v, ss1);
            dt1 = __builtin_fmaf(v, q[e], dt1);
          } else {
            ss0 = __builtin_fmaf(v, v, ss0);
            dt0 = __builtin_fmaf(v, q[e], dt0);
          }
        }
      }
    }
    float ss = wave_sum_to_lane63(ss0 + ss1);
    float dt = wave_sum_to_lane63(dt0 + dt1);
    ss = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ss), 63));
    dt = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, dt), 63));
    const float inv = __builtin_amdgcn_rsqf(ss * P.inv_d + P.eps);
    const float logit = dt * inv;
    if ((uint32_t)lane == s) {
      my_logit = logit;
      my_inv = inv;
    }

    // ---- online softmax over depth, rescale folded into the FMA ----
    // State at a token's first source: m = -inf, l = 0, acc = 0, so the
    // first source takes the "new maximum" path with c = exp(-inf) = 0.
    if (logit > m) {
      const float cf = __expf(m - logit);
      l = __builtin_fmaf(l, cf, 1.f);
      m = logit;
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          if constexpr (BF16) acc_rescale_add_bf16(acc[c][2 * w], acc[c][2 * w + 1], x[c][w], cf);
          else acc_rescale_add_f32(acc[c][w], x[c][w], cf);
        }
      }
    } else {
      const float pr = __expf(logit - m);
      l += pr;
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          if constexpr (BF16) acc_add_scaled_bf16(acc[c][2 * w], acc[c][2 * w + 1], x[c][w], pr);
          else acc_add_scaled_f32(acc[c][w], x[c][w], pr);
        }
      }
    }

    if (s == (uint32_t)(S - 1)) {
      // ---- finalize the token row ----
      const float rl = 1.0f / l;
      // The lane's part of the output row: OPC pieces of OPB bytes per chunk.
      u32x4 pk[NCH][OPC];
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        float o[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) o[e] = acc[c][e] * rl;
        if constexpr (OUTBF) {
          if constexpr (VEC == 8) {
            pk[c][0] = u32x4{pack_bf16(o[0], o[1]), pack_bf16(o[2], o[3]), pack_bf16(o[4], o[5]), pack_bf16(o[6], o[7])};
          } else {
            pk[c][0] = u32x4{pack_bf16(o[0], o[1]), pack_bf16(o[2], o[3]), 0u, 0u};
          }
        } else {
#pragma unroll
          for (int h = 0; h < OPC; ++h)
            pk[c][h] = u32x4{as_u32(o[4 * h]), as_u32(o[4 * h + 1]), as_u32(o[4 * h + 2]), as_u32(o[4 * h + 3])};
        }
      }
      if (!FUSED && batch > 1) {
        // stage the row; the wave's batch is stored when full (or at the end)
        if (nheld == 0) t_first = t;
        if (nheld < batch) {
#pragma unroll
          for (int c = 0; c < NCH; ++c) {
#pragma unroll
            for (int h = 0; h < OPC; ++h) {
              char* sp = stage_row(nheld) + ((c * OPC + h) * 64 + lane) * OPB;
              if constexpr (OPB == 16) *reinterpret_cast<u32x4*>(sp) = pk[c][h];
              else *reinterpret_cast<u32x2*>(sp) = u32x2{pk[c][h][0], pk[c][h][1]};
            }
          }
        } else {
          // register slot nheld - batch, selected with compile-time indices
#pragma unroll
          for (int r = 0; r < REG_ROWS; ++r) {
            if (nheld == batch + (uint32_t)r) {
#pragma unroll
              for (int c = 0; c < NCH; ++c) {
#pragma unroll
                for (int h = 0; h < OPC; ++h) held[r][c][h] = pk[c][h];
              }
            }
          }
        }
        nheld = __builtin_amdgcn_readfirstlane(nheld + 1);
        if (nheld == full_batch) {
          flush_staged();
          nheld = 0;
        }
      } else {
        const __amdgpu_buffer_rsrc_t orsrc = out_rsrc(t);
        const uint32_t lane_ob = lane_out_offset();
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
#pragma unroll
          for (int h = 0; h < OPC; ++h) {
            const uint32_t off = lane_ob + (uint32_t)(c * 64 * VEC * OES + 16 * h);
            if (nt_st) {
              if constexpr (OPB == 16) st_row_nt(orsrc, off, pk[c][h]);
              else st_row_nt(orsrc, off, u32x2{pk[c][h][0], pk[c][h][1]});
            } else {
              if constexpr (OPB == 16) st_row(orsrc, off, pk[c][h]);
              else st_row(orsrc, off, u32x2{pk[c][h][0], pk[c][h][1]});
            }
          }
        }
      }
      if (P.weights || P.logits || P.inv_rms || P.lse) {
        if (lane < S) {
          if (P.weights) P.weights[(int64_t)lane * P.n_tokens + t] = __expf(my_logit - m) * rl;
          if (P.logits) P.logits[(int64_t)t * S + lane] = my_logit;
          if (P.inv_rms) P.inv_rms[(int64_t)t * S + lane] = my_inv;
        }
        if (lane == 0 && P.lse) P.lse[t] = m + __logf(l);
      }
      m = -__builtin_inff();
      l = 0.f;
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc_zero(acc[c][e]);
      }
    }
  };

  // ---- two-slot pipeline over this wave's (token, source) items ----
  // The next item is requested as soon as the current one has arrived and
  // before the wave works on it: one row per wave in flight, its load
  // overlapping the work.  (Requesting it before the current row has
  // arrived, with up to two rows per wave in flight, measured 1.5-4 points
  // of peak slower at S >= 4, and the HBM then served three waves per CU
  // better than four.)  The prefetch is issued unconditionally (past the
  // last item it re-reads the current, valid row), with no branch around
  // the loads.
  using SlotA = std::integral_constant<int, 0>;
  using SlotB = std::integral_constant<int, 1>;
  // Items (row, source) of this wave in order; two per iteration so slot A
  // and slot B alternate.  A counted loop with one exit keeps the control
  // flow uniform (two break exits were structurised into divergent flow
  // variables, pulling the counters into VGPRs).
  const uint32_t rows_here = (n_tok - tok - 1) / nw + 1;
  const uint32_t n_items = rows_here * (uint32_t)S;
  auto advance = [&](uint32_t t, uint32_t ss, uint32_t& t_out, uint32_t& s_out) {
    const bool wrap = ss + 1 == (uint32_t)S;
    s_out = wrap ? 0u : ss + 1;
    t_out = wrap ? t + nw : t;
  };
  uint32_t s = 0;
  load_item(bufA, dX, tok, 0, 0u);
  for (uint32_t i = 0; i < n_items; i += 2) {
    const bool has1 = i + 1 < n_items;
    const bool has2 = i + 2 < n_items;
    uint32_t t1, s1, t2, s2;
    advance(tok, s, t1, s1);
    advance(t1, s1, t2, s2);
    // past the last item the prefetch re-reads the current (valid) row
    load_item(bufB, dX, has1 ? t1 : tok, has1 ? s1 : s, arrival_zero(bufA[NCH - 1][3]));
    process(bufA, dX, tok, s, SlotA{});
    load_item(bufA, dX, has2 ? t2 : tok, has2 ? s2 : s, arrival_zero(bufB[NCH - 1][3]));
    if (has1) process(bufB, dX, t1, s1, SlotB{});
    tok = __builtin_amdgcn_readfirstlane(t2);
    s = __builtin_amdgcn_readfirstlane(s2);
  }
  if constexpr (!FUSED) {
    if (nheld > 0) flush_staged();
  }
}


// ------------------------------------------------------- backward body --

// Source counts up to which the next row is loaded before the current row's
// gradients are stored (the prefetch holds a second copy of the row).
#ifndef ATTNRES_BWD_PREFETCH_MAX_S
#define ATTNRES_BWD_PREFETCH_MAX_S 4
#endif
//
// One workgroup per token row (grid-stride), thread i owning chunks
// i, i+blockDim, ... as in route_body.  The S source chunks and the output
// gradient G are held in registers (packed); per source the thread forms
// sum(x^2), x.qw and x.G, the 3S partial sums go through one DPP wave
// reduction + LDS exchange, and every thread then recomputes the softmax and
// writes its chunks of the S source gradients
//   dx_s = w_s G + c1_s qw + c2_s x_s,
//   c1_s = dl_s r_s,  c2_s = -dl_s l_s r_s^2 / D,  dl_s = w_s (g_lse + G.x_s - G.out).
// The next row's sources and G are loaded before the current row's gradients
// are stored, so a workgroup's loads overlap its own stores.  The query
// gradient sum_s c1_s x_s is accumulated in registers over all rows the
// workgroup handles and written once as this workgroup's partial.
// ADD: sources with a non-NULL P.dadd[s] get dx_s + dadd[s] (the addend chunk
// is requested before the chunk's products and added in fp32, one rounding;
// a source without an addend adds the 0 that an empty buffer resource reads).


template <int S, int V, bool BF16, bool GBF, bool ADD = false>
__device__ __forceinline__ void route_bwd_body(const attnres_route_bwd_params& P) {
  constexpr bool PF = S <= ATTNRES_BWD_PREFETCH_MAX_S;
  using C = Chunk<BF16>;
  constexpr int VEC = C::VEC;
  using GC = PackedChunk<VEC, GBF>;
  constexpr int NV = 3 * S;             // sum(x^2), x.qw, x.G per source
  constexpr int H2 = (NV + 3) / 4;
  constexpr int NP = 4 * H2;
  constexpr int SEG = S <= 8 ? 8 : 16;  // lanes of the softmax
  __shared__ float red[2][ATTNRES_KMAX_WAVES][NP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nwaves = (blockDim.x + 63) >> 6;

  // Where registers are tight (S >= 5) each thread's chunks of qw and, for
  // V == 1, of its running query-gradient sum live in (dynamic) LDS instead,
  // VEC floats per chunk; the LDS is thread-private, so no barrier.
  // Layout [chunk / 16][h][chunk % 16] (float4 h of a chunk's VEC floats):
  // sixteen consecutive lanes touch 256 contiguous bytes per access, so the
  // 128-bit LDS accesses are free of bank conflicts, and h is an immediate
  // offset.  Each array has a slot for every chunk index the block touches
  // (V * blockDim of them, a multiple of 16); the slots of chunks past the
  // row end hold zeros, so the dot loop reads them without a branch (stale
  // LDS there can be Inf or NaN, which 0 * x would carry into the row).
  constexpr bool QW_LDS = S >= 5;
  constexpr bool DQW_LDS = QW_LDS && V == 1;
  constexpr int NPL = VEC / 4;
  extern __shared__ float4 bwd_lds[];
  float4* s_qw = bwd_lds;
  float4* s_dqw = bwd_lds + (int)(V * blockDim.x) * NPL;
  auto lds_at = [](int c, int h) { return (c & ~15) * NPL + h * 16 + (c & 15); };
  float qw_reg[QW_LDS ? 1 : V][VEC];
  float dqw_reg[DQW_LDS ? 1 : V][VEC];
#pragma unroll
  for (int k = 0; k < (DQW_LDS ? 1 : V); ++k) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) dqw_reg[k][e] = 0.f;
  }

  int chunk[V];
  bool ok[V];
#pragma unroll
  for (int k = 0; k < V; ++k) {
    chunk[k] = tid + k * (int)blockDim.x;
    ok[k] = chunk[k] < P.nchunk;
    if (!ok[k]) {
      if constexpr (QW_LDS) {
#pragma unroll
        for (int h = 0; h < VEC / 4; ++h) s_qw[lds_at(chunk[k], h)] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
      continue;
    }
    const int64_t off = (int64_t)chunk[k] * VEC;
    float q[VEC];
    load_param<VEC>(P.query, off, P.param_bf16, q);
    if (P.gain != nullptr) {
      float g[VEC];
      load_param<VEC>(P.gain, off, P.param_bf16, g);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float prod = q[e] * g[e];
        q[e] = P.param_bf16 ? round_bf16(prod) : prod;
      }
    }
    if constexpr (QW_LDS) {
#pragma unroll
      for (int h = 0; h < VEC / 4; ++h) {
        s_qw[lds_at(chunk[k], h)] = make_float4(q[4 * h], q[4 * h + 1], q[4 * h + 2], q[4 * h + 3]);
        if constexpr (DQW_LDS) s_dqw[lds_at(chunk[k], h)] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) qw_reg[QW_LDS ? 0 : k][e] = q[e];
    }
  }
  auto qw_chunk = [&](int k, float (&q)[VEC]) {
    if constexpr (QW_LDS) {
#pragma unroll
      for (int h = 0; h < VEC / 4; ++h) {
        const float4 t = s_qw[lds_at(chunk[k], h)];
        q[4 * h] = t.x;
        q[4 * h + 1] = t.y;
        q[4 * h + 2] = t.z;
        q[4 * h + 3] = t.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) q[e] = ok[k] ? qw_reg[QW_LDS ? 0 : k][e] : 0.f;
    }
  };

  const int64_t row_bytes_ld = P.src_ld * C::BYTES;
  const int64_t grow_bytes_ld = P.gout_ld * (GBF ? 2 : 4);
  u32x4 x[S][V];
  GC g[V];
  auto load_row = [&](int64_t t) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const char* row = reinterpret_cast<const char*>(P.src[s]) + t * row_bytes_ld;
#pragma unroll
      for (int k = 0; k < V; ++k) x[s][k] = ok[k] ? ldg_global<u32x4>(row + (int64_t)chunk[k] * 16) : u32x4{0, 0, 0, 0};
    }
    const char* grow = reinterpret_cast<const char*>(P.grad_out) + t * grow_bytes_ld;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      if (ok[k]) g[k].load(grow, chunk[k]);
      else g[k].zero();
    }
  };

  int ph = 0;
  int64_t tok = blockIdx.x;
  if (tok < P.n_tokens) load_row(tok);
  for (; tok < P.n_tokens; tok += gridDim.x) {
    // ---- sum(x^2), x.qw, x.G per source ----
    float part[NP];
#pragma unroll
    for (int j = 0; j < NP; ++j) part[j] = 0.f;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      float q[VEC];
      qw_chunk(k, q);
#pragma unroll
      for (int s = 0; s < S; ++s) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float v = C::elem(x[s][k], e);
          part[s] = __builtin_fmaf(v, v, part[s]);
          part[S + s] = __builtin_fmaf(v, q[e], part[S + s]);
          part[2 * S + s] = __builtin_fmaf(v, g[k].elem(e), part[2 * S + s]);
        }
      }
    }
    // ---- transposing wave reduction, one LDS exchange ----
    wave_reduce_to_lds<H2>(part, red[ph][wave], lane);
    __syncthreads();

    // ---- softmax recomputed and the coefficients of dx, lane s per source ----
    const int ls = lane % SEG;
    const bool slot = ls < S;
    float t_ss = 0.f, t_dot = 0.f, t_gx = 0.f;
    if (slot) {
      for (int w = 0; w < nwaves; ++w) {
        t_ss += red[ph][w][ls];
        t_dot += red[ph][w][S + ls];
        t_gx += red[ph][w][2 * S + ls];
      }
    }
    ph ^= 1;
    const float rl = __builtin_amdgcn_rsqf(t_ss * P.inv_d + P.eps);
    const float ll = slot ? t_dot * rl : -__builtin_inff();
    const float m = seg_max<SEG>(ll);
    const float el = slot ? __expf(ll - m) : 0.f;
    const float wl = el * (1.0f / seg_sum<SEG>(el));
    const float go = seg_sum<SEG>(wl * t_gx);  // G . out = sum_s w_s (G . x_s)
    const float glse = P.grad_lse != nullptr ? P.grad_lse[tok] : 0.f;
    // glse is added after G.x_s - G.out cancels: added to G.x_s first it would
    // be rounded to the ulp of that (much larger) dot product
    const float c1l = wl * (glse + (t_gx - go)) * rl;
    const float c2l = -c1l * ll * rl * P.inv_d;
    // The coefficients are the same in every lane: scalar registers.
    float c1[S], c2[S], wgt[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
      wgt[s] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), s));
      c1[s] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, c1l), s));
      c2[s] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, c2l), s));
    }

    // ---- keep this row, start loading the next one ----
    u32x4 xc[S][V];
    GC gc[V];
#pragma unroll
    for (int k = 0; k < V; ++k) {
#pragma unroll
      for (int s = 0; s < S; ++s) xc[s][k] = x[s][k];
      gc[k] = g[k];
    }
    const int64_t next = tok + gridDim.x;
    if (PF && next < P.n_tokens) load_row(next);

    // ---- write the source gradients, accumulate the query gradient ----
    // The packed rows are re-expanded here rather than kept as fp32 from the
    // first pass (that would double the register footprint of the sources).
#pragma unroll
    for (int s = 0; s < S; ++s) {
#pragma unroll
      for (int k = 0; k < V; ++k) asm volatile("" : "+v"(xc[s][k]));
    }
#pragma unroll
    for (int k = 0; k < V; ++k) {
      if (!ok[k]) continue;
      float q[VEC], acc[VEC];
      qw_chunk(k, q);
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
#pragma unroll
      for (int s = 0; s < S; ++s) {
        char* drow = reinterpret_cast<char*>(P.dsrc[s]) + tok * P.dsrc_ld * C::BYTES;
        const __amdgpu_buffer_rsrc_t drsrc = row_rsrc(drow, (uint32_t)(P.d * C::BYTES));
        // ADD: the addend chunk through a buffer resource over its row, empty
        // (loads return 0, no memory access) when the source has no addend,
        // so the code has no branch
        u32x4 ad = u32x4{0, 0, 0, 0};
        if constexpr (ADD) {
          const void* abase = P.dadd[s];
          char* arow = reinterpret_cast<char*>(const_cast<void*>(abase)) + tok * P.dsrc_ld * C::BYTES;
          ad = ld_row(row_rsrc(arow, abase != nullptr ? (uint32_t)(P.d * C::BYTES) : 0u), (uint32_t)chunk[k] * 16);
        }
        float dx[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float v = C::elem(xc[s][k], e);
          dx[e] = __builtin_fmaf(c2[s], v, __builtin_fmaf(c1[s], q[e], wgt[s] * gc[k].elem(e)));
          acc[e] = __builtin_fmaf(c1[s], v, acc[e]);
        }
        if constexpr (ADD) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) dx[e] += C::elem(ad, e);
        }
        if constexpr (BF16) {
          st_row_nt(drsrc, (uint32_t)chunk[k] * 16,
                    u32x4{pack_bf16(dx[0], dx[1]), pack_bf16(dx[2], dx[3]), pack_bf16(dx[4], dx[5]),
                          pack_bf16(dx[6], dx[7])});
        } else {
          st_row_nt(drsrc, (uint32_t)chunk[k] * 16,
                    u32x4{as_u32(dx[0]), as_u32(dx[1]), as_u32(dx[2]), as_u32(dx[3])});
        }
      }
      if constexpr (DQW_LDS) {
#pragma unroll
        for (int h = 0; h < VEC / 4; ++h) {
          float4 t = s_dqw[lds_at(chunk[k], h)];
          t.x += acc[4 * h];
          t.y += acc[4 * h + 1];
          t.z += acc[4 * h + 2];
          t.w += acc[4 * h + 3];
          s_dqw[lds_at(chunk[k], h)] = t;
        }
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) dqw_reg[DQW_LDS ? 0 : k][e] += acc[e];
      }
    }
    if (!PF && next < P.n_tokens) load_row(next);
  }

  // ---- this workgroup's query-gradient partial ----
  float4* prow = reinterpret_cast<float4*>(P.dqw_part + (int64_t)blockIdx.x * P.d);
#pragma unroll
  for (int k = 0; k < V; ++k) {
    if (!ok[k]) continue;
#pragma unroll
    for (int h = 0; h < VEC / 4; ++h) {
      if constexpr (DQW_LDS) {
        prow[chunk[k] * (VEC / 4) + h] = s_dqw[lds_at(chunk[k], h)];
      } else {
        const float* a = dqw_reg[DQW_LDS ? 0 : k];
        prow[chunk[k] * (VEC / 4) + h] = make_float4(a[4 * h], a[4 * h + 1], a[4 * h + 2], a[4 * h + 3]);
      }
    }
  }
}

// ------------------------------------------ row-per-wave routing backward --
//
// The routing backward with one wave per token row, for bf16 sources and
// output gradients and rows of NCH KiB (hidden = 512 * NCH): a resident grid
// of one workgroup per CU whose waves take rows grid-stride.  A row's items
// stream through the two-slot pipeline of the forward streaming kernel (the
// next item is requested as soon as the current one has arrived): G, then
// x_0 .. x_{S-1}.  Per source the lane forms sum(x^2) and x.G (v_dot2 on the
// packed words) and x.qw (fp32 qw from LDS) over its chunks, three DPP wave
// sums give the row's values, and the packed source row is kept in registers
// ((S - KL) * NCH * 4 of them, which at one wave per SIMD the compiler places
// partly in the accumulation half of the register file) or, for the first KL
// sources, in the wave's part of the LDS.  After the last source the softmax
// and the coefficients are formed wave-uniformly, and each gradient row
//   dx_s = w_s G + c1_s qw + c2_s x_s,
//   c1_s = dl_s r_s,  c2_s = -dl_s l_s r_s^2 / D,  dl_s = w_s (g_lse + G.x_s - G.out),
// is stored whole, source after source, while the next row's G is in flight.
// The query gradient sum_s c1_s x_s accumulates per lane over the wave's
// rows; at the end the workgroup's waves add theirs through LDS in a fixed
// order and write one fp32 partial row per workgroup, as route_bwd_body does.
// KL > 0: the first KL source rows are kept in the wave's part of the
// dynamic LDS instead of registers (more sources than the registers hold).
// ADD: sources with a non-NULL P.dadd[s] get dx_s + dadd[s]; the addend row
// of source s + 1 is requested before the gradient of source s is formed, so
// one addend row per wave is in flight behind the row being stored.
// DEFER (with ADD): only the last source's gradient row is formed (plus
// dadd[S-1], requested before the second pass); for sources 0 .. S-2 lane s
// stores the token's (w_s, c1_s, c2_s, 0) to P.coef, and workgroup 0 writes
// the folded query to P.qfold (bf16 parameters), so that the sum of a
// block's gradients over the points that read it is formed once, later
// (route_bwd_gather_seg_body), from the points' output gradients.
template <int S, int NCH, int KL, bool ADD = false, bool DEFER = false>
__device__ __forceinline__ void route_bwd_stream_body(const attnres_route_bwd_params& P) {
  static_assert(KL >= 0 && KL < S, "at least one source row is kept in registers");
  static_assert(!DEFER || (ADD && S >= 2), "deferred gradients need a committed source and the addend path");
  // Dynamic LDS in float4 slots [chunk][half][lane] (consecutive lanes 16
  // bytes apart): the folded query in fp32 and, past it, each wave's KL kept
  // rows ([wave][row][chunk][lane], 16-byte slots); at the end one row of
  // query-gradient sums per wave from the start.
  extern __shared__ float4 bws_lds[];
  constexpr int ROW4 = NCH * 2 * 64;  // float4 slots of one row
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nwv = (int)(blockDim.x >> 6);
  auto slot = [&](int c, int h) { return (c * 2 + h) * 64 + lane; };

  // ---- folded query (query * gain, rounded to the parameter dtype) ----
  for (int i = tid; i < NCH * 64; i += (int)blockDim.x) {
    float q[8];
    load_param<8>(P.query, (int64_t)i * 8, P.param_bf16, q);
    if (P.gain != nullptr) {
      float gn[8];
      load_param<8>(P.gain, (int64_t)i * 8, P.param_bf16, gn);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float prod = q[e] * gn[e];
        q[e] = P.param_bf16 ? round_bf16(prod) : prod;
      }
    }
    const int c = i >> 6, l = i & 63;
    if constexpr (DEFER) {
      // bf16 parameters: the folded query is bf16-exact and kept packed
      const u32x4 pk = {pack_bf16(q[0], q[1]), pack_bf16(q[2], q[3]), pack_bf16(q[4], q[5]), pack_bf16(q[6], q[7])};
      reinterpret_cast<u32x4*>(bws_lds)[c * 64 + l] = pk;
      if (blockIdx.x == 0) stg<u32x4>(static_cast<char*>(P.qfold) + (size_t)i * 16, pk);
    } else {
      bws_lds[(c * 2) * 64 + l] = make_float4(q[0], q[1], q[2], q[3]);
      bws_lds[(c * 2 + 1) * 64 + l] = make_float4(q[4], q[5], q[6], q[7]);
    }
  }
  __syncthreads();
  // The query is read from LDS at each use (an opaque index): hoisted out of
  // the row loop it would hold 8 * NCH more registers.
  auto qw_chunk = [&](int c, float (&q)[8]) {
    int i0 = slot(c, 0);
    asm volatile("" : "+v"(i0));
    const float4 qa = bws_lds[i0], qb = bws_lds[i0 + 64];
    q[0] = qa.x, q[1] = qa.y, q[2] = qa.z, q[3] = qa.w;
    q[4] = qb.x, q[5] = qb.y, q[6] = qb.z, q[7] = qb.w;
  };
  // DEFER: the packed chunk (x.qw then on v_dot2 like the x.x and x.G sums)
  auto qp_chunk = [&](int c) {
    int i0 = c * 64 + lane;
    asm volatile("" : "+v"(i0));
    return reinterpret_cast<const u32x4*>(bws_lds)[i0];
  };
  auto lane63 = [](float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
  };

  float dq[NCH][8];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
#pragma unroll
    for (int e = 0; e < 8; ++e) dq[c][e] = 0.f;
  }
  // 32-bit wave-uniform row counters (scalar loop control, as in stream_body)
  const uint32_t n_tok = (uint32_t)P.n_tokens;
  const uint32_t nw = gridDim.x * (uint32_t)nwv;
  const uint32_t tok0 = blockIdx.x * (uint32_t)nwv + (uint32_t)wave;
  if (tok0 < n_tok) {  // no barrier inside: waves without rows go straight to the partial sums
    const uint64_t row_bytes = (uint64_t)P.src_ld * 2;
    const uint64_t grow_bytes = (uint64_t)P.gout_ld * 2;
    const uint64_t drow_bytes = (uint64_t)P.dsrc_ld * 2;
    const uint64_t gout0 = reinterpret_cast<uint64_t>(P.grad_out);
    const uint32_t lane_off = (uint32_t)lane * 16;
    // z: an arrival_zero() of the previous item, added to the lane offsets
    auto load_row = [&](u32x4(&buf)[NCH], uint64_t addr, uint32_t z) {
      const char* row = uniform_ptr(addr);
#pragma unroll
      for (int c = 0; c < NCH; ++c) buf[c] = ldg_global<u32x4>(row + (lane_off + (uint32_t)(c * 1024) + z));
      // keep the prefetch ahead of the work on the current row
      __builtin_amdgcn_sched_barrier(0);
    };
    u32x4 gnext[NCH], g[NCH], xa[NCH], xb[NCH], keep[S - KL][NCH];
    u32x4* kept_lds = reinterpret_cast<u32x4*>(bws_lds) + ROW4 + (wave * KL) * NCH * 64 + lane;
    const uint32_t rows = (n_tok - tok0 - 1) / nw + 1;
    uint32_t t = tok0;
    load_row(gnext, gout0 + (uint64_t)t * grow_bytes, 0u);
    for (uint32_t r = 0; r < rows; ++r) {
      t = __builtin_amdgcn_readfirstlane(t);
#pragma unroll
      for (int c = 0; c < NCH; ++c) g[c] = gnext[c];
      load_row(xa, reinterpret_cast<uint64_t>(P.src[0]) + (uint64_t)t * row_bytes, arrival_zero(g[NCH - 1][3]));
      float lg[S], ri[S], gx[S];
#pragma unroll
      for (int s = 0; s < S; ++s) {
        u32x4(&cur)[NCH] = (s & 1) ? xb : xa;
        u32x4(&nxt)[NCH] = (s & 1) ? xa : xb;
        const uint32_t z = arrival_zero(cur[NCH - 1][3]);
        if (s + 1 < S) {
          load_row(nxt, reinterpret_cast<uint64_t>(P.src[s + 1]) + (uint64_t)t * row_bytes, z);
        } else {
          // the next row's G (past the wave's last row, this row's G again)
          const uint32_t tn = r + 1 < rows ? t + nw : t;
          load_row(gnext, gout0 + (uint64_t)tn * grow_bytes, z);
        }
        // ---- sum(x^2), x.G and x.qw over this lane's chunks (two chains each) ----
        float ss0 = 0.f, ss1 = 0.f, gx0 = 0.f, gx1 = 0.f, dt0 = 0.f, dt1 = 0.f;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
          if constexpr (DEFER) {
            const u32x4 qp = qp_chunk(c);
#pragma unroll
            for (int w = 0; w < 4; ++w) {
              const uint32_t xw = cur[c][w];
              if (w & 1) {
                ss1 = dot2_bf16(xw, xw, ss1);
                gx1 = dot2_bf16(xw, g[c][w], gx1);
                dt1 = dot2_bf16(xw, qp[w], dt1);
              } else {
                ss0 = dot2_bf16(xw, xw, ss0);
                gx0 = dot2_bf16(xw, g[c][w], gx0);
                dt0 = dot2_bf16(xw, qp[w], dt0);
              }
            }
          } else {
            float q[8];
            qw_chunk(c, q);
#pragma unroll
            for (int w = 0; w < 4; ++w) {
              const uint32_t xw = cur[c][w];
              if (w & 1) {
                ss1 = dot2_bf16(xw, xw, ss1);
                gx1 = dot2_bf16(xw, g[c][w], gx1);
              } else {
                ss0 = dot2_bf16(xw, xw, ss0);
                gx0 = dot2_bf16(xw, g[c][w], gx0);
              }
              dt0 = __builtin_fmaf(bf_lo(xw), q[2 * w], dt0);
              dt1 = __builtin_fmaf(bf_hi(xw), q[2 * w + 1], dt1);
            }
          }
          if (s < KL) kept_lds[(s * NCH + c) * 64] = cur[c];
          else keep[s >= KL ? s - KL : 0][c] = cur[c];
        }
        const float ss = lane63(wave_sum_to_lane63(ss0 + ss1));
        const float dt = lane63(wave_sum_to_lane63(dt0 + dt1));
        gx[s] = lane63(wave_sum_to_lane63(gx0 + gx1));
        ri[s] = __builtin_amdgcn_rsqf(ss * P.inv_d + P.eps);
        lg[s] = dt * ri[s];
      }

      // ---- softmax over the sources and the coefficients (wave-uniform) ----
      float m = lg[0];
#pragma unroll
      for (int s = 1; s < S; ++s) m = lg[s] > m ? lg[s] : m;
      float ex[S], sum = 0.f;
#pragma unroll
      for (int s = 0; s < S; ++s) {
        ex[s] = __expf(lg[s] - m);
        sum += ex[s];
      }
      const float rsum = 1.0f / sum;
      float wgt[S], go = 0.f;  // go = G . out = sum_s w_s (G . x_s)
#pragma unroll
      for (int s = 0; s < S; ++s) {
        wgt[s] = ex[s] * rsum;
        go = __builtin_fmaf(wgt[s], gx[s], go);
      }
      // dL/dlse through the scalar cache (a wave-uniform read-only value): a
      // vector load here would be waited for with the next row's G, which is
      // in flight behind it, and put G's round trip into every row's chain
      const float glse = P.grad_lse != nullptr ? ld_scalar_f32(P.grad_lse + t) : 0.f;
      float c1[S], c2[S];
#pragma unroll
      for (int s = 0; s < S; ++s) {
        // glse is added after G.x_s - G.out cancels (added to G.x_s first it
        // would be rounded to the ulp of that much larger dot product)
        c1[s] = wgt[s] * (glse + (gx[s] - go)) * ri[s];
        c2[s] = -c1[s] * lg[s] * ri[s] * P.inv_d;
      }
      if constexpr (DEFER) {
        // the committed sources' coefficients: lane s holds source s's record
        float4 rec = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int s = 0; s < S - 1; ++s) {
          if (lane == s) rec = make_float4(wgt[s], c1[s], c2[s], 0.f);
        }
        char* crow = const_cast<char*>(uniform_ptr(reinterpret_cast<uint64_t>(P.coef) + (uint64_t)t * ((S - 1) * 16)));
        // lanes >= S-1 fall outside the resource's range: their stores are dropped
        st_row_nt(row_rsrc(crow, (uint32_t)((S - 1) * 16)), lane_off,
                  u32x4{as_u32(rec.x), as_u32(rec.y), as_u32(rec.z), as_u32(rec.w)});
      }

      // ---- the gradient rows, one whole row per source ----
      // The kept rows are re-expanded here (opaque copies) rather than kept
      // unpacked from the first pass, which would double their registers.
      // Addend rows through a buffer resource over the row, empty (loads
      // return 0 without a memory access) for a source without an addend, so
      // the loop has no branch.
      u32x4 adA[ADD ? NCH : 1], adB[ADD ? NCH : 1];
      auto load_add = [&](u32x4(&buf)[ADD ? NCH : 1], int s) {
        const void* abase = P.dadd[s];
        char* row = const_cast<char*>(uniform_ptr(reinterpret_cast<uint64_t>(abase) + (uint64_t)t * drow_bytes));
        const __amdgpu_buffer_rsrc_t ar = row_rsrc(row, abase != nullptr ? (uint32_t)(NCH * 1024) : 0u);
#pragma unroll
        for (int c = 0; c < (ADD ? NCH : 1); ++c) buf[c] = ld_row(ar, lane_off + (uint32_t)(c * 1024));
      };
      if constexpr (ADD) load_add(adA, DEFER ? S - 1 : 0);
#pragma unroll
      for (int s = 0; s < S; ++s) {
        u32x4(&ad_cur)[ADD ? NCH : 1] = (DEFER || !(s & 1)) ? adA : adB;
        u32x4(&ad_nxt)[ADD ? NCH : 1] = (s & 1) ? adA : adB;
        if constexpr (ADD && !DEFER) {
          if (s + 1 < S) load_add(ad_nxt, s + 1 < S ? s + 1 : 0);
        }
        u32x4 xk[NCH];
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
          if (s < KL) {
            xk[c] = kept_lds[(s * NCH + c) * 64];
          } else {
            xk[c] = keep[s >= KL ? s - KL : 0][c];
            asm volatile("" : "+v"(xk[c]));
          }
        }
        if (DEFER && s < S - 1) {
          // a committed source: its query-gradient term only
#pragma unroll
          for (int c = 0; c < NCH; ++c) {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
              dq[c][2 * w] = __builtin_fmaf(c1[s], bf_lo(xk[c][w]), dq[c][2 * w]);
              dq[c][2 * w + 1] = __builtin_fmaf(c1[s], bf_hi(xk[c][w]), dq[c][2 * w + 1]);
            }
          }
          continue;
        }
        char* drow = const_cast<char*>(uniform_ptr(reinterpret_cast<uint64_t>(P.dsrc[s]) + (uint64_t)t * drow_bytes));
        const __amdgpu_buffer_rsrc_t dr = row_rsrc(drow, (uint32_t)(NCH * 1024));
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
          float q[8];
          if constexpr (DEFER) {
            const u32x4 qp = qp_chunk(c);
#pragma unroll
            for (int w = 0; w < 4; ++w) q[2 * w] = bf_lo(qp[w]), q[2 * w + 1] = bf_hi(qp[w]);
          } else {
            qw_chunk(c, q);
          }
          u32x4 pk;
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const uint32_t xw = xk[c][w], gw = g[c][w];
            const float x0 = bf_lo(xw), x1 = bf_hi(xw);
            float d0 = __builtin_fmaf(c2[s], x0, __builtin_fmaf(c1[s], q[2 * w], wgt[s] * bf_lo(gw)));
            float d1 = __builtin_fmaf(c2[s], x1, __builtin_fmaf(c1[s], q[2 * w + 1], wgt[s] * bf_hi(gw)));
            dq[c][2 * w] = __builtin_fmaf(c1[s], x0, dq[c][2 * w]);
            dq[c][2 * w + 1] = __builtin_fmaf(c1[s], x1, dq[c][2 * w + 1]);
            if constexpr (ADD) {
              d0 += bf_lo(ad_cur[c][w]);
              d1 += bf_hi(ad_cur[c][w]);
            }
            pk[w] = pack_bf16(d0, d1);
          }
          st_row_nt(dr, lane_off + (uint32_t)(c * 1024), pk);
        }
      }
      t += nw;
    }
  }

  // ---- this workgroup's query-gradient partial: the waves' sums through LDS ----
  __syncthreads();  // every wave is done with the query in LDS
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
      bws_lds[wave * ROW4 + slot(c, h)] =
          make_float4(dq[c][4 * h], dq[c][4 * h + 1], dq[c][4 * h + 2], dq[c][4 * h + 3]);
  }
  __syncthreads();
  float4* prow = reinterpret_cast<float4*>(P.dqw_part + (int64_t)blockIdx.x * P.d);
  for (int j = tid; j < ROW4; j += (int)blockDim.x) {
    float4 a = bws_lds[j];
    for (int w = 1; w < nwv; ++w) {
      const float4 b = bws_lds[w * ROW4 + j];
      a.x += b.x;
      a.y += b.y;
      a.z += b.z;
      a.w += b.w;
    }
    const int c = j >> 7, h = (j >> 6) & 1, l = j & 63;
    prow[(c * 64 + l) * 2 + h] = a;
  }
}


// Non-temporal row load: a row read once.
__device__ __forceinline__ u32x4 ld_row_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2);
}

// ------------------------------------------- segment of deferred sums --
//
// The gradients of blocks 0 .. NB-1 from the terms of the points that read
// them all (the points between two commits), each point's dL/dout row read
// once.  A wave takes one part of a token row (CPW KiB of the NCH KiB) at a
// time, a unit, and streams its items through a ring of DEPTH slots (the
// next item requested once the oldest in flight has arrived): per term its
// record row (lane j: block j's (w, c1, c2)), its dL/dout part and its
// folded query part; per block its running sum part and x-coefficient sum;
// with P.final_block the last block's x and addend parts.  Every item is
// one accumulation on the matrix cores (v_mfma_f32_4x4x4_16b_bf16) into the
// blocks' fp32 sums of the unit,
//   acc_j += a_j G + b_j Q
// (per element and group of four blocks one product: lane 4b+i of A carries
// block 4s+i's (a hi, b hi, a lo, b lo), the coefficients split into bf16
// hi + lo parts, hi + lo equal to the fp32 value to about 2^-17 of it; lane
// 4b+j's B column its own element (G, Q, G, Q); D element i is block 4s+i
// at that element):
//   term p:      G = dL/dout_p, Q = q_p,  a_j = w_pj,  b_j = c1_pj,
//                cs_j += c2_pj (lane j);
//   block k:     G = its running sum, a_k = 1, cs_k += its x-coefficient sum;
//   final:       G = x, Q = addend,  a_L = cs_L, b_L = 1  (L = NB - 1),
// so the accumulation runs the same code for every item.  After the unit's
// last item the blocks' sums are stored (bf16, non-temporal; with
// P.final_block the last one as the block's gradient) and, for the blocks
// that carry on, cs_j to csum_out.
template <int NB, int NCH, int CPW, int DEPTH>
__device__ __forceinline__ void route_bwd_gather_seg_body(const attnres_route_bwd_gather_seg_params& P) {
  static_assert(NCH % CPW == 0, "a row splits into whole parts");
  static_assert(NB >= 1 && NB <= 8, "blocks of one segment");
  static_assert(DEPTH >= 2, "one item in flight behind the one processed");
  constexpr uint32_t PARTS = NCH / CPW;
  constexpr uint32_t PB = CPW * 1024;  // bytes of one part of a row
  constexpr int R = (NB + 3) / 4;      // groups of four blocks
  constexpr int L = NB - 1;
  const int lane = threadIdx.x & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t nwv = (uint32_t)P.block >> 6;
  const uint32_t n_items = (uint32_t)P.n_tokens * PARTS;
  const uint32_t nw = gridDim.x * nwv;
  const uint32_t item0 = blockIdx.x * nwv + wave;
  if (item0 >= n_items) return;
  const uint32_t rows = (n_items - item0 - 1) / nw + 1;  // units of this wave
  const uint32_t nt = (uint32_t)P.num_terms;
  const bool fin = P.final_block != 0;
  // terms, then one item per block, then (final) the last block's x and addend
  const uint32_t per = nt + NB + (fin ? 1u : 0u);
  const uint32_t lane_off = (uint32_t)lane * 16;

  // item (j, r) of the wave's units into a slot: every item issues the same
  // loads into the same registers (one record load, CPW B and CPW A parts;
  // empty resources read zeros), so the wait for a slot counts exactly the
  // loads issued after it.  The record load takes 12 bytes (w, c1, c2): a
  // loaded register left unused would be reused while its load is in flight,
  // and overwriting it waits for that load.
  auto issue = [&](u32x4(&a)[CPW], u32x4(&b)[CPW], u32x3& rec, uint32_t j, uint32_t r, uint32_t z) {
    if (j >= rows) {
      j = rows - 1;
      r = per - 1;
    }
    j = __builtin_amdgcn_readfirstlane(j);
    r = __builtin_amdgcn_readfirstlane(r);
    const uint32_t item = item0 + j * nw;
    const uint64_t t = item / PARTS;
    const uint32_t h = item % PARTS;
    char* abase = nullptr;
    char* bbase = nullptr;
    char* cbase = nullptr;
    uint32_t abytes = 0, bbytes = 0, cbytes = 0, coff = 0;
    if (r < nt) {
      const attnres_gather_term& T = P.term[r];
      abase = const_cast<char*>(uniform_ptr(reinterpret_cast<uint64_t>(T.grad_out) + t * (uint64_t)P.gout_ld * 2 + h * PB));
      bbase = const_cast<char*>(static_cast<const char*>(T.qfold)) + h * PB;
      cbase = const_cast<char*>(uniform_ptr(reinterpret_cast<uint64_t>(T.coef) + t * (uint64_t)T.coef_ld * 4));
      abytes = bbytes = PB;
      cbytes = NB * 16;  // lane j: block j's record
      coff = lane_off;
    } else if (r < nt + NB) {
      // the block's running sum part and (record word 0, every lane) its x-coefficient sum
      const void* pin = P.blk[r - nt].part_in;
      const float* cin = P.blk[r - nt].csum_in;
      abase = const_cast<char*>(uniform_ptr(reinterpret_cast<uint64_t>(pin) + t * (uint64_t)P.out_ld * 2 + h * PB));
      abytes = pin != nullptr ? PB : 0u;
      cbase = const_cast<char*>(uniform_ptr(reinterpret_cast<uint64_t>(cin) + t * 4));
      cbytes = cin != nullptr ? 4u : 0u;
    } else {
      abase = const_cast<char*>(uniform_ptr(reinterpret_cast<uint64_t>(P.x) + t * (uint64_t)P.x_ld * 2 + h * PB));
      bbase = const_cast<char*>(uniform_ptr(reinterpret_cast<uint64_t>(P.addend) + t * (uint64_t)P.out_ld * 2 + h * PB));
      abytes = PB;
      bbytes = P.addend != nullptr ? PB : 0u;
    }
    const __amdgpu_buffer_rsrc_t rc = row_rsrc(cbase, cbytes);
    const __amdgpu_buffer_rsrc_t rb = row_rsrc(bbase, bbytes);
    const __amdgpu_buffer_rsrc_t ra = row_rsrc(abase, abytes);
    // records and the B part first: loads return in order, so the A part's arrival implies theirs
    rec = __builtin_amdgcn_raw_buffer_load_b96(rc, coff + z, 0, 0);
#pragma unroll
    for (int c = 0; c < CPW; ++c) b[c] = __builtin_amdgcn_raw_buffer_load_b128(rb, lane_off + (uint32_t)(c * 1024) + z, 0, 0);
#pragma unroll
    for (int c = 0; c < CPW; ++c) a[c] = ld_row_nt(ra, lane_off + (uint32_t)(c * 1024) + z);
    __builtin_amdgcn_sched_barrier(0);
  };

  // block k's sum at element e of chunk c: element k % 4 of acc[k / 4][c][e]
  f32x4 acc[R][CPW][8];
#pragma unroll
  for (int g = 0; g < R; ++g) {
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][c][e] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  float csl = 0.f;  // lane k: block k's x-coefficient sum
  auto lane_f = [](uint32_t v, int l) { return as_f32(__builtin_amdgcn_readlane(v, l)); };
  auto process = [&](u32x4(&a)[CPW], u32x4(&b)[CPW], const u32x3& rec, uint32_t j, uint32_t r) {
    // the A operands: (a, b) of block 4g + (lane & 3), split hi + lo
    float av[R], bv[R];
    if (r < nt) {
#pragma unroll
      for (int g = 0; g < R; ++g) {
        const int src = (4 * g + (lane & 3)) << 2;
        av[g] = as_f32(__builtin_amdgcn_ds_bpermute(src, (int)rec[0]));
        bv[g] = as_f32(__builtin_amdgcn_ds_bpermute(src, (int)rec[1]));
      }
      csl += as_f32(rec[2]);
    } else {
      const bool blk = r < nt + NB;
      const uint32_t kb = blk ? r - nt : (uint32_t)L;
      const float ka = blk ? 1.f : lane_f(as_u32(csl), L);
      const float kq = blk ? 0.f : 1.f;
#pragma unroll
      for (int g = 0; g < R; ++g) {
        const bool mine = (uint32_t)(4 * g + (lane & 3)) == kb;
        av[g] = mine ? ka : 0.f;
        bv[g] = mine ? kq : 0.f;
      }
      if (blk) csl += (uint32_t)lane == kb ? as_f32(rec[0]) : 0.f;
    }
    u32x2 am[R];
#pragma unroll
    for (int g = 0; g < R; ++g) {
      const uint32_t hi = pack_bf16(av[g], bv[g]);
      am[g] = u32x2{hi, pack_bf16(av[g] - bf_lo(hi), bv[g] - bf_hi(hi))};
    }
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t pl = __builtin_amdgcn_perm(b[c][q], a[c][q], 0x05040100u);  // (G, Q) of element 2q
        const uint32_t ph = __builtin_amdgcn_perm(b[c][q], a[c][q], 0x07060302u);  // of element 2q + 1
#pragma unroll
        for (int g = 0; g < R; ++g) {
          acc[g][c][2 * q] = mfma_4x4x4(am[g], u32x2{pl, pl}, acc[g][c][2 * q]);
          acc[g][c][2 * q + 1] = mfma_4x4x4(am[g], u32x2{ph, ph}, acc[g][c][2 * q + 1]);
        }
      }
    }
    if (r != per - 1) return;
    // the unit's last item: store every block's sum, clear them
    const uint32_t item = item0 + j * nw;
    const uint64_t t = item / PARTS;
    const uint32_t h = item % PARTS;
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      char* orow = const_cast<char*>(
          uniform_ptr(reinterpret_cast<uint64_t>(P.blk[k].part_out) + t * (uint64_t)P.out_ld * 2 + h * PB));
      const __amdgpu_buffer_rsrc_t ro = row_rsrc(orow, PB);
#pragma unroll
      for (int c = 0; c < CPW; ++c) {
        u32x4 pk;
#pragma unroll
        for (int q = 0; q < 4; ++q) pk[q] = pack_bf16(acc[k / 4][c][2 * q][k % 4], acc[k / 4][c][2 * q + 1][k % 4]);
        st_row_nt_hidden(ro, lane_off + (uint32_t)(c * 1024), pk);
      }
      if (k < L || !fin) {
        const float csk = lane_f(as_u32(csl), k);
        if (h == 0 && lane == 0) st_f32_hidden(P.blk[k].csum_out + t, csk);
      }
    }
#pragma unroll
    for (int g = 0; g < R; ++g) {
#pragma unroll
      for (int c = 0; c < CPW; ++c) {
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][c][e] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
    csl = 0.f;
  };
  auto after = [per](uint32_t& j, uint32_t& r) {
    const uint32_t r1 = r + 1;
    const bool wrap = r1 == per;
    r = __builtin_amdgcn_readfirstlane(wrap ? 0u : r1);
    j = __builtin_amdgcn_readfirstlane(wrap ? j + 1 : j);
  };

  u32x4 A[DEPTH][CPW], B[DEPTH][CPW];
  u32x3 Rc[DEPTH];
  uint32_t ji = 0, ri = 0, jp = 0, rp = 0;
#pragma unroll
  for (int u = 0; u < DEPTH - 1; ++u) {
    issue(A[u], B[u], Rc[u], ji, ri, 0u);
    after(ji, ri);
  }
  const uint32_t items = rows * per;
  // whole rounds of the ring without conditions (each wait then counts the
  // loads issued after it across the loop's back edge), then the last,
  // partial round
  uint32_t i = 0;
  for (; i + DEPTH <= items; i += DEPTH) {
#pragma unroll
    for (int u = 0; u < DEPTH; ++u) {
      const int nx = (u + DEPTH - 1) % DEPTH;  // the slot processed last, refilled now
      issue(A[nx], B[nx], Rc[nx], ji, ri, arrival_zero(A[u][CPW - 1][3]));
      after(ji, ri);
      process(A[u], B[u], Rc[u], jp, rp);
      after(jp, rp);
    }
  }
#pragma unroll
  for (int u = 0; u < DEPTH - 1; ++u) {
    if (i + (uint32_t)u < items) {
      process(A[u], B[u], Rc[u], jp, rp);
      after(jp, rp);
    }
  }
}

// ------------------------------------------- batched-query backward body --
//
// Backward of Q >= 2 queries over one set of sources (the batched phase-1
// call, ops/phase_1.py:88-284 with NUM_QUERIES_PER_BLOCK > 1), one pass over
// the sources.  One workgroup per token row (grid-stride), chunks as in
// route_bwd_body; the S source chunks stay in registers for all queries.  Per
// query q: x.qw_q and x.G_q per source (sum(x^2) once per row), the
// transposing wave reduction and one LDS exchange, the softmax and the
// coefficients lane-parallel (lane s per source), then
//   acc_s  += w_qs G_q + c1_qs qw_q      (fp32 registers)
//   c2sum_s += c2_qs                      (lane s)
// and once per row dx_s = acc_s + c2sum_s x_s.  c1_qs goes to `c1`
// (n_tokens, Q, S): the query gradients sum_rows sum_s c1_qs x_s are formed by
// route_bwd_dqw_body in a second pass over the sources.

template <int VEC>
__device__ __forceinline__ void load_qw_ptr(const void* query, const void* gain, bool bf16, int q, int d, int chunk,
                                            float (&qw)[VEC]) {
  const int64_t off = (int64_t)chunk * VEC;
  load_param<VEC>(query, (int64_t)q * d + off, bf16, qw);
  if (gain != nullptr) {
    float g[VEC];
    load_param<VEC>(gain, off, bf16, g);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float prod = qw[e] * g[e];
      qw[e] = bf16 ? round_bf16(prod) : prod;
    }
  }
}

template <int S, int V, bool BF16, bool GBF>
__device__ __forceinline__ void route_bwd_mq_body(const attnres_route_bwd_mq_params& P) {
  using C = Chunk<BF16>;
  constexpr int VEC = C::VEC;
  using GC = PackedChunk<VEC, GBF>;
  constexpr int NV = 3 * S;  // sum(x^2), x.qw_q, x.G_q per source
  constexpr int H2 = (NV + 3) / 4;
  constexpr int NP = 4 * H2;
  constexpr int SEG = S <= 8 ? 8 : 16;
  __shared__ float red[2][ATTNRES_KMAX_WAVES][NP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int block = P.block;
  const int nwaves = (block + 63) >> 6;
  const int nq = P.num_queries;

  int chunk[V];
  bool ok[V];
#pragma unroll
  for (int k = 0; k < V; ++k) {
    chunk[k] = tid + k * block;
    ok[k] = chunk[k] < P.nchunk;
  }

  // Source rows through buffer resources: a chunk past the row end reads 0
  // and its gradient store is dropped.
  const int64_t row_bytes_ld = P.src_ld * C::BYTES;
  const uint32_t row_bytes = (uint32_t)(P.d * C::BYTES);
  u32x4 x[S][V];
  auto load_row = [&](int64_t t) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      char* row = reinterpret_cast<char*>(const_cast<void*>(P.src[s])) + t * row_bytes_ld;
      const __amdgpu_buffer_rsrc_t rs = row_rsrc(row, row_bytes);
#pragma unroll
      for (int k = 0; k < V; ++k) x[s][k] = ld_row(rs, (uint32_t)chunk[k] * 16);
    }
  };

  const int ls = lane % SEG;  // the source of this lane in the softmax
  const bool slot = ls < S;
  const int64_t grow_bytes_ld = P.gout_ld * (GBF ? 2 : 4);
  const int64_t gq_bytes = P.gout_qstride * (GBF ? 2 : 4);
  float gain_reg[V][VEC];  // the norm gain of the fold, once per thread
#pragma unroll
  for (int k = 0; k < V; ++k) {
    if (P.gain != nullptr && ok[k]) {
      load_param<VEC>(P.gain, (int64_t)chunk[k] * VEC, P.param_bf16, gain_reg[k]);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) gain_reg[k][e] = 1.f;
    }
  }

  int ph = 0;
  if ((int64_t)blockIdx.x < P.n_tokens) load_row(blockIdx.x);
  for (int64_t tok = blockIdx.x; tok < P.n_tokens; tok += gridDim.x) {
    float ssp[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
      ssp[s] = 0.f;
#pragma unroll
      for (int k = 0; k < V; ++k) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float v = C::elem(x[s][k], e);
          ssp[s] = __builtin_fmaf(v, v, ssp[s]);
        }
      }
    }
    float acc[S][V][VEC];
#pragma unroll
    for (int s = 0; s < S; ++s) {
#pragma unroll
      for (int k = 0; k < V; ++k) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[s][k][e] = 0.f;
      }
    }
    float c2sum = 0.f;

    // The next query's output-gradient and query chunks are requested before
    // the current query is processed (one query ahead), so the per-query
    // loads overlap the previous query's reduction and accumulation.
    GC gn[V];
    ParamRaw<VEC> qn[V];
    auto fetch_query = [&](int q) {
      const char* grow = reinterpret_cast<const char*>(P.grad_out) + q * gq_bytes + tok * grow_bytes_ld;
#pragma unroll
      for (int k = 0; k < V; ++k) {
        if (ok[k]) {
          gn[k].load(grow, chunk[k]);
          load_param_raw<VEC>(reinterpret_cast<const char*>(P.query) + (int64_t)q * P.d * (P.param_bf16 ? 2 : 4),
                              chunk[k], P.param_bf16, qn[k]);
        } else {
          gn[k].zero();
          qn[k].w[0] = u32x4{0, 0, 0, 0};
          if constexpr (VEC == 8) qn[k].w[1] = u32x4{0, 0, 0, 0};
        }
      }
    };
    fetch_query(0);
    for (int q = 0; q < nq; ++q) {
      // ---- this query's folded query and output-gradient chunks ----
      float qw[V][VEC];
      GC g[V];
#pragma unroll
      for (int k = 0; k < V; ++k) {
        g[k] = gn[k];
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float qv = param_elem<VEC>(qn[k], e, P.param_bf16);
          if (P.gain != nullptr) {
            const float prod = qv * gain_reg[k][e];
            qw[k][e] = P.param_bf16 ? round_bf16(prod) : prod;
          } else {
            qw[k][e] = qv;
          }
        }
      }
      if (q + 1 < nq) fetch_query(q + 1);

      // ---- sum(x^2), x.qw_q, x.G_q; transposing reduction; one exchange ----
      float part[NP];
#pragma unroll
      for (int j = 0; j < NP; ++j) part[j] = j < S ? ssp[j] : 0.f;
#pragma unroll
      for (int k = 0; k < V; ++k) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            const float v = C::elem(x[s][k], e);
            part[S + s] = __builtin_fmaf(v, qw[k][e], part[S + s]);
            part[2 * S + s] = __builtin_fmaf(v, g[k].elem(e), part[2 * S + s]);
          }
        }
      }
      wave_reduce_to_lds<H2>(part, red[ph][wave], lane);
      __syncthreads();

      // ---- softmax and coefficients, lane s per source ----
      float t_ss = 0.f, t_dot = 0.f, t_gx = 0.f;
      if (slot) {
        for (int w = 0; w < nwaves; ++w) {
          t_ss += red[ph][w][ls];
          t_dot += red[ph][w][S + ls];
          t_gx += red[ph][w][2 * S + ls];
        }
      }
      ph ^= 1;
      const float rl = __builtin_amdgcn_rsqf(t_ss * P.inv_d + P.eps);
      const float ll = slot ? t_dot * rl : -__builtin_inff();
      const float m = seg_max<SEG>(ll);
      const float el = slot ? __expf(ll - m) : 0.f;
      const float wl = el * (1.0f / seg_sum<SEG>(el));
      const float go = seg_sum<SEG>(wl * t_gx);  // G_q . out_q
      const float glse = P.grad_lse != nullptr ? P.grad_lse[(int64_t)q * P.n_tokens + tok] : 0.f;
      const float c1l = slot ? wl * (glse + (t_gx - go)) * rl : 0.f;  // cancel first, then add glse
      c2sum += slot ? -c1l * ll * rl * P.inv_d : 0.f;
      if (wave == 0 && lane < S) P.c1[(tok * nq + q) * S + lane] = c1l;
      float wgt[S], c1[S];
#pragma unroll
      for (int s = 0; s < S; ++s) {
        wgt[s] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), s));
        c1[s] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, c1l), s));
      }
#pragma unroll
      for (int s = 0; s < S; ++s) {
#pragma unroll
        for (int k = 0; k < V; ++k) {
#pragma unroll
          for (int e = 0; e < VEC; ++e)
            acc[s][k][e] = __builtin_fmaf(wgt[s], g[k].elem(e), __builtin_fmaf(c1[s], qw[k][e], acc[s][k][e]));
        }
      }
    }

    // ---- dx_s = acc_s + c2sum_s x_s, stored once ----
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const float c2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, c2sum), s));
      char* drow = reinterpret_cast<char*>(P.dsrc[s]) + tok * P.dsrc_ld * C::BYTES;
      const __amdgpu_buffer_rsrc_t drs = row_rsrc(drow, row_bytes);
#pragma unroll
      for (int k = 0; k < V; ++k) {
        float dx[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) dx[e] = __builtin_fmaf(c2, C::elem(x[s][k], e), acc[s][k][e]);
        if constexpr (BF16) {
          st_row_nt(drs, (uint32_t)chunk[k] * 16,
                 u32x4{pack_bf16(dx[0], dx[1]), pack_bf16(dx[2], dx[3]), pack_bf16(dx[4], dx[5]),
                       pack_bf16(dx[6], dx[7])});
        } else {
          st_row_nt(drs, (uint32_t)chunk[k] * 16, u32x4{as_u32(dx[0]), as_u32(dx[1]), as_u32(dx[2]), as_u32(dx[3])});
        }
      }
    }
    if (tok + gridDim.x < P.n_tokens) load_row(tok + gridDim.x);
  }
}

// ------------------------------- batched-query backward on the matrix cores --
//
// The source gradients of the batched-query routing for bf16 sources, bf16
// output gradients and bf16 parameters with Q <= 4*NQ4 queries (the serving
// engine's phase 1 under autograd).  One workgroup per row (grid-stride),
// thread i owning chunks i, i+block, ...; per row the S source chunks and
// the output-gradient chunks of every query are loaded once (the next row's
// after the current row's stores), the folded queries sit in dynamic LDS.
// Per group of four queries:
//  * x.qw_q and x.G_q per (query, source) with v_dot2_f32_bf16 (sum(x^2) in
//    the first group), reduced by the transposing tree, one LDS exchange;
//  * lane 8g + s runs the softmax of query g over the sources and forms
//      w_qs, c1_qs = w_qs (g_lse + G_q.x_s - G_q.out_q) r_s,
//      c2_qs = -c1_qs l_qs r_s / D
//    (G_q.out_q = sum_s w_qs G_q.x_s, from the reduced values);
//  * w and c1 move into MFMA A operands (ds_bpermute): lane 4b+i carries
//    source 4ks+i of a group of four sources, the four queries along k, as
//    bf16 hi + lo parts.
// Then per chunk and element the matrix cores form
//   dx_s = sum_q (w_qs G_q + c1_qs qw_q)
// for four sources at a time (v_mfma_f32_4x4x4_16b_bf16 with B = the
// lane's own G_q / qw_q at that element, four queries along k), the VALU
// adds (sum_q c2_qs) x_s and each gradient row is written once.  c1 goes to
// the workspace for the query-gradient pass (route_bwd_dqw_body).
template <int S, int V, int NQ4>
__device__ __forceinline__ void route_bwd_mqg_body(const attnres_route_bwd_mq_params& P) {
  constexpr int VEC = 8;
  constexpr int SEG = 8;                 // lanes per query in the softmax (S <= 8)
  constexpr int KS = (S + 3) / 4;        // groups of four sources
  constexpr int NQ = 4 * NQ4;            // query slots
  // per group two reductions: sum(x^2) and x.qw of 4 queries (5S values),
  // then x.G of 4 queries (4S values), so fewer partial sums are live at once
  constexpr int HA = (5 * S + 3) / 4, HB = S;
  constexpr int NPA = 4 * HA, NPB = 4 * HB;
  static_assert(S >= 1 && S <= SEG, "one softmax lane per (query, source)");
  __shared__ float red[2][ATTNRES_KMAX_WAVES][NPA + NPB];
  // packed folded queries, zero past the batch, laid out [chunk / 16][query slot][chunk % 16]:
  // sixteen consecutive lanes read 256 contiguous bytes (no LDS bank conflicts)
  // and a thread's queries sit at immediate offsets of 256 bytes from one address
  extern __shared__ u32x4 qg_lds[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int block = P.block;
  const int nwaves = (block + 63) >> 6;
  const int nq = P.num_queries;
  const int nchunk = P.nchunk;

  auto qslot = [](int c) { return (c & ~15) * NQ + (c & 15); };  // query q at + 16 * q
  int chunk[V];
  const u32x4* qrow[V];  // this thread's chunks of the staged queries: qrow[k][16 * q], q < NQ
#pragma unroll
  for (int k = 0; k < V; ++k) {
    chunk[k] = tid + k * block;
    qrow[k] = qg_lds + qslot(chunk[k] < nchunk ? chunk[k] : nchunk - 1);  // chunks past the end read zeros
  }

  // ---- the folded queries into LDS, once per workgroup (consecutive threads
  // read consecutive chunks of one query) ----
  for (int i = tid; i < NQ * nchunk; i += block) {
    const int q = i / nchunk, c = i % nchunk;
    float t[VEC];
    if (q < nq) {
      load_qw_ptr<VEC>(P.query, P.gain, true, q, P.d, c, t);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) t[e] = 0.f;
    }
    qg_lds[qslot(c) + 16 * q] =
        u32x4{pack_bf16(t[0], t[1]), pack_bf16(t[2], t[3]), pack_bf16(t[4], t[5]), pack_bf16(t[6], t[7])};
  }

  // Rows through buffer resources: a chunk past the row end reads 0 and its
  // gradient store is dropped; query slots past the batch hold zeros.
  const int64_t row_bytes_ld = P.src_ld * 2;
  const uint32_t row_bytes = (uint32_t)(P.d * 2);
  u32x4 x[S][V], gq[NQ][V];
  auto load_row = [&](int64_t t) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      char* row = reinterpret_cast<char*>(const_cast<void*>(P.src[s])) + t * row_bytes_ld;
      const __amdgpu_buffer_rsrc_t rs = row_rsrc(row, row_bytes);
#pragma unroll
      for (int k = 0; k < V; ++k) x[s][k] = ld_row(rs, (uint32_t)chunk[k] * 16);
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      char* grow = reinterpret_cast<char*>(const_cast<void*>(P.grad_out)) + (q * P.gout_qstride + t * P.gout_ld) * 2;
      const __amdgpu_buffer_rsrc_t rg = row_rsrc(grow, q < nq ? row_bytes : 0u);
#pragma unroll
      for (int k = 0; k < V; ++k) gq[q][k] = ld_row(rg, (uint32_t)chunk[k] * 16);
    }
  };
  if ((int64_t)blockIdx.x < P.n_tokens) load_row(blockIdx.x);

  __syncthreads();

  int ph = 0;
  for (int64_t tok = blockIdx.x; tok < P.n_tokens; tok += gridDim.x) {
    // Lane-derived indices and addresses are recomputed per row from an
    // opaque copy of the lane id: hoisted out of the row loop they stayed
    // live across it and spilled.
    int lr = lane;
    asm volatile("" : "+v"(lr));
    const int sg = lr / SEG, ss = lr % SEG;  // softmax lane: query sg of the group, source ss
    const int ai = lr & 3;                   // A-operand row: source 4*ks + ai
    u32x2 awh[NQ4][KS], awl[NQ4][KS], ach[NQ4][KS], acl[NQ4][KS];
    float c2acc = 0.f;
    float rl = 0.f;  // 1/rms of source ss, from the first group's reduction
#pragma unroll
    for (int g4 = 0; g4 < NQ4; ++g4) {
      const int q0 = 4 * g4;
      // ---- sum(x^2) (first group), x.qw and x.G of four queries, packed dot products, two reductions ----
      {
        float part[NPA];
#pragma unroll
        for (int j = 0; j < NPA; ++j) part[j] = 0.f;
        if (g4 == 0) {
#pragma unroll
          for (int k = 0; k < V; ++k) {
#pragma unroll
            for (int s = 0; s < S; ++s) {
#pragma unroll
              for (int w = 0; w < 4; ++w) part[s] = dot2_bf16(x[s][k][w], x[s][k][w], part[s]);
            }
          }
        }
#pragma unroll
        for (int k = 0; k < V; ++k) {
          u32x4 qv[4];
#pragma unroll
          for (int g = 0; g < 4; ++g) qv[g] = qrow[k][16 * (q0 + g)];
#pragma unroll
          for (int s = 0; s < S; ++s) {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
#pragma unroll
              for (int g = 0; g < 4; ++g) part[S + g * S + s] = dot2_bf16(x[s][k][w], qv[g][w], part[S + g * S + s]);
            }
          }
        }
        wave_reduce_to_lds<HA>(part, red[ph][wave], lr);
      }
      {
        float part[NPB];
#pragma unroll
        for (int j = 0; j < NPB; ++j) part[j] = 0.f;
#pragma unroll
        for (int k = 0; k < V; ++k) {
#pragma unroll
          for (int s = 0; s < S; ++s) {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
#pragma unroll
              for (int g = 0; g < 4; ++g) part[g * S + s] = dot2_bf16(x[s][k][w], gq[q0 + g][k][w], part[g * S + s]);
            }
          }
        }
        wave_reduce_to_lds<HB>(part, red[ph][wave] + NPA, lr);
      }
      __syncthreads();

      // ---- softmax and coefficients, lane 8g + s ----
      const int q = q0 + sg;
      const bool slot = sg < 4 && ss < S && q < nq;
      float t_ss = 0.f, t_dot = 0.f, t_gx = 0.f;
      if (slot) {
        for (int w = 0; w < nwaves; ++w) {
          if (g4 == 0) t_ss += red[ph][w][ss];
          t_dot += red[ph][w][S + sg * S + ss];
          t_gx += red[ph][w][NPA + sg * S + ss];
        }
      }
      ph ^= 1;
      if (g4 == 0) rl = __builtin_amdgcn_rsqf(t_ss * P.inv_d + P.eps);
      const float ll = slot ? t_dot * rl : -__builtin_inff();
      const float m = seg_max<SEG>(ll);
      const float el = slot ? __expf(ll - m) : 0.f;
      const float sum = seg_sum<SEG>(el);
      const float wl = slot ? el * (1.0f / sum) : 0.f;
      const float go = seg_sum<SEG>(wl * t_gx);  // G_q . out_q
      const float glse = slot && P.grad_lse != nullptr ? P.grad_lse[(int64_t)q * P.n_tokens + tok] : 0.f;
      const float c1l = slot ? wl * (glse + (t_gx - go)) * rl : 0.f;  // cancel first, then add glse
      c2acc += slot ? -c1l * ll * rl * P.inv_d : 0.f;
      if (wave == 0 && slot) P.c1[(tok * nq + q) * S + ss] = c1l;

      // ---- A operands: source 4*ks + ai, queries q0 .. q0+3 along k ----
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int src_s = 4 * ks + ai;
        float wv[4], cv[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int from = (g * SEG + src_s) * 4;
          wv[g] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(from, __builtin_bit_cast(int, wl)));
          cv[g] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(from, __builtin_bit_cast(int, c1l)));
          if (src_s >= S) wv[g] = cv[g] = 0.f;
        }
        const uint32_t w01 = pack_bf16(wv[0], wv[1]), w23 = pack_bf16(wv[2], wv[3]);
        const uint32_t c01 = pack_bf16(cv[0], cv[1]), c23 = pack_bf16(cv[2], cv[3]);
        awh[g4][ks] = u32x2{w01, w23};
        awl[g4][ks] = u32x2{pack_bf16(wv[0] - bf_lo(w01), wv[1] - bf_hi(w01)),
                            pack_bf16(wv[2] - bf_lo(w23), wv[3] - bf_hi(w23))};
        ach[g4][ks] = u32x2{c01, c23};
        acl[g4][ks] = u32x2{pack_bf16(cv[0] - bf_lo(c01), cv[1] - bf_hi(c01)),
                            pack_bf16(cv[2] - bf_lo(c23), cv[3] - bf_hi(c23))};
      }
    }

    // sum over the queries of c2_qs, per source (lanes 8g + s)
    float c2s[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
      float t = 0.f;
#pragma unroll
      for (int g = 0; g < 4; ++g)
        t += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, c2acc), g * SEG + s));
      c2s[s] = t;
    }
    // ---- dx_s = sum_q (w_qs G_q + c1_qs qw_q) + c2_s x_s, per chunk, group of
    // four sources and element pair: the two accumulators of a pair are rounded
    // and packed as soon as its queries are summed, so a source group holds 16
    // packed words, not 32 fp32 sums ----
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const uint32_t* qword = reinterpret_cast<const uint32_t*>(qrow[k]);  // query q, word w at [64 q + w]
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        uint32_t packed[4][4];  // packed[i][w]: elements 2w, 2w+1 of source 4*ks + i
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int g4 = 0; g4 < NQ4; ++g4) {
            const int q0 = 4 * g4;
            uint32_t qv[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) qv[g] = qword[64 * (q0 + g) + w];
            // B operands of elements 2w (low halves) and 2w+1 (high halves), four queries along k
            const u32x2 bgl = {__builtin_amdgcn_perm(gq[q0 + 1][k][w], gq[q0][k][w], 0x05040100u),
                               __builtin_amdgcn_perm(gq[q0 + 3][k][w], gq[q0 + 2][k][w], 0x05040100u)};
            const u32x2 bgh = {__builtin_amdgcn_perm(gq[q0 + 1][k][w], gq[q0][k][w], 0x07060302u),
                               __builtin_amdgcn_perm(gq[q0 + 3][k][w], gq[q0 + 2][k][w], 0x07060302u)};
            const u32x2 bql = {__builtin_amdgcn_perm(qv[1], qv[0], 0x05040100u),
                               __builtin_amdgcn_perm(qv[3], qv[2], 0x05040100u)};
            const u32x2 bqh = {__builtin_amdgcn_perm(qv[1], qv[0], 0x07060302u),
                               __builtin_amdgcn_perm(qv[3], qv[2], 0x07060302u)};
            lo = mfma_4x4x4(awh[g4][ks], bgl, lo);
            hi = mfma_4x4x4(awh[g4][ks], bgh, hi);
            lo = mfma_4x4x4(awl[g4][ks], bgl, lo);
            hi = mfma_4x4x4(awl[g4][ks], bgh, hi);
            lo = mfma_4x4x4(ach[g4][ks], bql, lo);
            hi = mfma_4x4x4(ach[g4][ks], bqh, hi);
            lo = mfma_4x4x4(acl[g4][ks], bql, lo);
            hi = mfma_4x4x4(acl[g4][ks], bqh, hi);
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int s = 4 * ks + i;
            if (s >= S) break;
            packed[i][w] = pack_bf16(__builtin_fmaf(c2s[s], bf_lo(x[s][k][w]), lo[i]),
                                     __builtin_fmaf(c2s[s], bf_hi(x[s][k][w]), hi[i]));
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int s = 4 * ks + i;
          if (s >= S) break;
          char* drow = reinterpret_cast<char*>(P.dsrc[s]) + tok * P.dsrc_ld * 2;
          st_row_nt(row_rsrc(drow, row_bytes), (uint32_t)chunk[k] * 16,
                 u32x4{packed[i][0], packed[i][1], packed[i][2], packed[i][3]});
        }
      }
    }
    if (tok + gridDim.x < P.n_tokens) load_row(tok + gridDim.x);
  }
}

// Query-gradient partials of the batched backward: each workgroup sums
// c1_qs x_s over its rows (grid-stride) and sources for up to 8 queries
// q0 .. q0+7 and writes them as its row of `part` (gridDim.x, Q, d).  Source
// chunks are requested four at a time.
template <int V, bool BF16>
__device__ __forceinline__ void route_bwd_dqw_body(const attnres_route_bwd_dqw_params& P) {
  using C = Chunk<BF16>;
  constexpr int VEC = C::VEC;
  constexpr int QG = 8;
  const int tid = threadIdx.x;
  const int block = P.block;
  const int S = P.num_sources;
  const int nq = P.num_queries;
  const int q0 = P.q0;
  const int ng = nq - q0 < QG ? nq - q0 : QG;

  int chunk[V];
  bool ok[V];
#pragma unroll
  for (int k = 0; k < V; ++k) {
    chunk[k] = tid + k * block;
    ok[k] = chunk[k] < P.nchunk;
  }
  float acc[QG][V][VEC];
#pragma unroll
  for (int g = 0; g < QG; ++g) {
#pragma unroll
    for (int k = 0; k < V; ++k) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[g][k][e] = 0.f;
    }
  }
  const int64_t row_bytes_ld = P.src_ld * C::BYTES;
  const uint32_t row_bytes = (uint32_t)(P.d * C::BYTES);
  constexpr int SG = 4;  // sources requested together
  for (int64_t tok = blockIdx.x; tok < P.n_tokens; tok += gridDim.x) {
    const float* crow = P.c1 + (tok * nq + q0) * S;
    for (int s0 = 0; s0 < S; s0 += SG) {
      u32x4 x[SG][V];
#pragma unroll
      for (int i = 0; i < SG; ++i) {
        const int s = s0 + i < S ? s0 + i : S - 1;  // past S: a repeated row, weight 0 below
        char* row = reinterpret_cast<char*>(const_cast<void*>(P.src[s])) + tok * row_bytes_ld;
        const __amdgpu_buffer_rsrc_t rs = row_rsrc(row, row_bytes);
#pragma unroll
        for (int k = 0; k < V; ++k) x[i][k] = ld_row(rs, (uint32_t)chunk[k] * 16);
      }
#pragma unroll
      for (int i = 0; i < SG; ++i) {
#pragma unroll
        for (int g = 0; g < QG; ++g) {
          const float c = (g < ng && s0 + i < S) ? crow[g * S + s0 + i] : 0.f;
#pragma unroll
          for (int k = 0; k < V; ++k) {
#pragma unroll
            for (int e = 0; e < VEC; ++e) acc[g][k][e] = __builtin_fmaf(c, C::elem(x[i][k], e), acc[g][k][e]);
          }
        }
      }
    }
  }
  float* prow = P.part + (int64_t)blockIdx.x * nq * P.d;
#pragma unroll
  for (int g = 0; g < QG; ++g) {
    if (g >= ng) break;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      if (!ok[k]) continue;
      float4* dst = reinterpret_cast<float4*>(prow + (int64_t)(q0 + g) * P.d + (int64_t)chunk[k] * VEC);
#pragma unroll
      for (int h = 0; h < VEC / 4; ++h)
        dst[h] = make_float4(acc[g][k][4 * h], acc[g][k][4 * h + 1], acc[g][k][4 * h + 2], acc[g][k][4 * h + 3]);
    }
  }
}


// Query-gradient partials on the matrix cores (bf16 sources): as
// route_bwd_dqw_body, with sum c1_qs x_s formed per element as column j of a
// 4x4x4 block product: A = c1 of four queries (lane 4b+i: query
// q0 + 4*g4 + i) over four (row, source) pairs (k), as bf16 hi + lo parts;
// B = the lane's own chunks of those four pairs at that element.  The
// workgroup's pairs (its rows grid-stride, each row's S sources in order) are
// taken four at a time whatever S is, so every k slot carries a real row (at
// S = 1 four rows, at S = 5 a row and a quarter); the next four pairs' chunks
// and c1 values are requested before the current four's 2 * 2 MFMAs per
// element (two query groups, hi and lo).  Slots past the last pair read
// through a zero-byte buffer resource: zeros, no memory traffic.
template <int V>
__device__ __forceinline__ void route_bwd_dqwm_body(const attnres_route_bwd_dqw_params& P) {
  constexpr int NQ4 = 2;  // eight queries per pass
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int block = P.block;
  const int S = P.num_sources;
  const int nq = P.num_queries;
  const int q0 = P.q0;
  const int ng = nq - q0 < 4 * NQ4 ? nq - q0 : 4 * NQ4;
  const int ai = lane & 3;

  int chunk[V];
  bool ok[V];
#pragma unroll
  for (int k = 0; k < V; ++k) {
    chunk[k] = tid + k * block;
    ok[k] = chunk[k] < P.nchunk;
  }
  f32x4 acc[V][8][NQ4];  // element h of chunk k, queries q0 + 4*g4 + i in acc[k][h][g4][i]
#pragma unroll
  for (int k = 0; k < V; ++k) {
#pragma unroll
    for (int h = 0; h < 8; ++h) {
#pragma unroll
      for (int g4 = 0; g4 < NQ4; ++g4) acc[k][h][g4] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  const int64_t row_bytes_ld = P.src_ld * 2;
  const uint32_t row_bytes = (uint32_t)(P.d * 2);
  const uint32_t rows =
      (int64_t)blockIdx.x < P.n_tokens ? (uint32_t)((P.n_tokens - 1 - blockIdx.x) / gridDim.x + 1) : 0u;
  const uint32_t npairs = rows * (uint32_t)S;
  const uint32_t items = (npairs + 3) / 4;

  // the next pair to request: row blockIdx.x + pj * gridDim.x, source ps
  uint32_t pj = 0, ps = 0, pnext = 0;
  auto load_item = [&](u32x4 (&x)[4][V], float (&c)[NQ4][4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool valid = pnext < npairs;
      const int64_t tok = (int64_t)blockIdx.x + (int64_t)pj * gridDim.x;
      char* row = reinterpret_cast<char*>(const_cast<void*>(P.src[ps])) + tok * row_bytes_ld;
      const __amdgpu_buffer_rsrc_t rs = row_rsrc(row, valid ? row_bytes : 0u);
#pragma unroll
      for (int k = 0; k < V; ++k) x[i][k] = ld_row(rs, (uint32_t)chunk[k] * 16);
      const float* crow = P.c1 + (tok * nq + q0) * S + ps;  // c1 of query q0 + g at crow[g * S]
#pragma unroll
      for (int g4 = 0; g4 < NQ4; ++g4) {
        const int g = 4 * g4 + ai;
        c[g4][i] = (valid && g < ng) ? crow[g * S] : 0.f;
      }
      ++pnext;
      if (++ps == (uint32_t)S) {
        ps = 0;
        ++pj;
      }
    }
  };

  u32x4 xa[4][V], xb[4][V];
  float ca[NQ4][4], cb[NQ4][4];
  if (items > 0) load_item(xa, ca);
  for (uint32_t it = 0; it < items; ++it) {
    if (it + 1 < items) load_item(xb, cb);
    u32x2 ah[NQ4], al[NQ4];
#pragma unroll
    for (int g4 = 0; g4 < NQ4; ++g4) {
      const float* c = ca[g4];
      const uint32_t h01 = pack_bf16(c[0], c[1]), h23 = pack_bf16(c[2], c[3]);
      ah[g4] = u32x2{h01, h23};
      al[g4] = u32x2{pack_bf16(c[0] - bf_lo(h01), c[1] - bf_hi(h01)), pack_bf16(c[2] - bf_lo(h23), c[3] - bf_hi(h23))};
    }
#pragma unroll
    for (int k = 0; k < V; ++k) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const u32x2 blo = {__builtin_amdgcn_perm(xa[1][k][w], xa[0][k][w], 0x05040100u),
                           __builtin_amdgcn_perm(xa[3][k][w], xa[2][k][w], 0x05040100u)};
        const u32x2 bhi = {__builtin_amdgcn_perm(xa[1][k][w], xa[0][k][w], 0x07060302u),
                           __builtin_amdgcn_perm(xa[3][k][w], xa[2][k][w], 0x07060302u)};
#pragma unroll
        for (int g4 = 0; g4 < NQ4; ++g4) {
          acc[k][2 * w][g4] = mfma_4x4x4(al[g4], blo, mfma_4x4x4(ah[g4], blo, acc[k][2 * w][g4]));
          acc[k][2 * w + 1][g4] = mfma_4x4x4(al[g4], bhi, mfma_4x4x4(ah[g4], bhi, acc[k][2 * w + 1][g4]));
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int k = 0; k < V; ++k) xa[i][k] = xb[i][k];
    }
#pragma unroll
    for (int g4 = 0; g4 < NQ4; ++g4) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) ca[g4][kk] = cb[g4][kk];
    }
  }
  float* prow = P.part + (int64_t)blockIdx.x * nq * P.d;
#pragma unroll
  for (int k = 0; k < V; ++k) {
    if (!ok[k]) continue;
#pragma unroll
    for (int g4 = 0; g4 < NQ4; ++g4) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int g = 4 * g4 + i;
        if (g >= ng) continue;
        float4* dst = reinterpret_cast<float4*>(prow + (int64_t)(q0 + g) * P.d + (int64_t)chunk[k] * 8);
        dst[0] = make_float4(acc[k][0][g4][i], acc[k][1][g4][i], acc[k][2][g4][i], acc[k][3][g4][i]);
        dst[1] = make_float4(acc[k][4][g4][i], acc[k][5][g4][i], acc[k][6][g4][i], acc[k][7][g4][i]);
      }
    }
  }
}

// ------------------------------------------------ merge backward body --

// VEC consecutive elements of a bf16 or fp32 row as fp32 (chunk = VEC elements).
template <bool BF, int VEC>
__device__ __forceinline__ void load_f32_chunk(const char* row, int chunk, float (&v)[VEC]) {
  if constexpr (BF) {
    if constexpr (VEC == 8) {
      const u32x4 t = ldg_global<u32x4>(row + (int64_t)chunk * 16);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        v[2 * w] = bf_lo(t[w]);
        v[2 * w + 1] = bf_hi(t[w]);
      }
    } else {
      const u32x2 t = ldg_global<u32x2>(row + (int64_t)chunk * 8);
      v[0] = bf_lo(t[0]);
      v[1] = bf_hi(t[0]);
      v[2] = bf_lo(t[1]);
      v[3] = bf_hi(t[1]);
    }
  } else {
#pragma unroll
    for (int h = 0; h < VEC / 4; ++h) {
      const u32x4 t = ldg_global<u32x4>(row + ((int64_t)chunk * VEC + 4 * h) * 4);
#pragma unroll
      for (int w = 0; w < 4; ++w) v[4 * h + w] = as_f32(t[w]);
    }
  }
}

// Store VEC fp32 values as one chunk of a bf16 or fp32 row.
template <bool BF, int VEC>
__device__ __forceinline__ void store_f32_chunk(__amdgpu_buffer_rsrc_t r, int chunk, const float (&o)[VEC]) {
  if constexpr (BF) {
    if constexpr (VEC == 8) {
      st_row_nt(r, (uint32_t)chunk * 16,
                u32x4{pack_bf16(o[0], o[1]), pack_bf16(o[2], o[3]), pack_bf16(o[4], o[5]), pack_bf16(o[6], o[7])});
    } else {
      st_row_nt(r, (uint32_t)chunk * 8, u32x2{pack_bf16(o[0], o[1]), pack_bf16(o[2], o[3])});
    }
  } else {
#pragma unroll
    for (int h = 0; h < VEC / 4; ++h)
      st_row_nt(r, (uint32_t)(chunk * VEC + 4 * h) * 4,
                u32x4{as_u32(o[4 * h]), as_u32(o[4 * h + 1]), as_u32(o[4 * h + 2]), as_u32(o[4 * h + 3])});
  }
}

// Backward of the phase-2 merge out = inter + pi (p - inter),
// pi = sigmoid(logit - lse), logit = (p.q) r, r = rsqrt(mean(p^2) + eps).
// With G = dL/dout, a = G.(p - inter) and gl = pi (1 - pi) a = dL/dlogit:
//   dinter = (1 - pi) G,   dlse = -gl,
//   dp = pi G + gl r q - gl logit r^2 / D p,   dq = sum over rows of gl r p.
// One workgroup per row as merge_body; the query gradient is accumulated in
// registers and written as this workgroup's partial (reduced by
// attnres_reduce_dqw_cols, or attnres_reduce_dqw_stage then attnres_reduce_dqw).
template <int V, bool PBF16, bool IBF16>
__device__ __forceinline__ void merge_bwd_body(const attnres_merge_bwd_params& P) {
  using C = Chunk<PBF16>;
  constexpr int VEC = C::VEC;
  __shared__ float red[2][ATTNRES_KMAX_WAVES][4];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nwaves = (blockDim.x + 63) >> 6;
  constexpr int IB = IBF16 ? 2 : 4;

  int chunk[V];
  bool ok[V];
  float qw[V][VEC];
  float dqa[V][VEC];
#pragma unroll
  for (int k = 0; k < V; ++k) {
    chunk[k] = tid + k * (int)blockDim.x;
    ok[k] = chunk[k] < P.nchunk;
    if (ok[k]) {
      load_param<VEC>(P.query, (int64_t)chunk[k] * VEC, P.param_bf16, qw[k]);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) qw[k][e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) dqa[k][e] = 0.f;
  }

  int ph = 0;
  for (int64_t tok = blockIdx.x; tok < P.n_tokens; tok += gridDim.x) {
    const char* prow = reinterpret_cast<const char*>(P.partial) + tok * (int64_t)P.d * C::BYTES;
    const char* irow = reinterpret_cast<const char*>(P.inter) + tok * (int64_t)P.d * IB;
    const char* grow = reinterpret_cast<const char*>(P.grad_out) + tok * (int64_t)P.d * IB;
    u32x4 p[V];
    float iv[V][VEC], gv[V][VEC];
#pragma unroll
    for (int k = 0; k < V; ++k) {
      if (ok[k]) {
        p[k] = ldg_global<u32x4>(prow + (int64_t)chunk[k] * 16);
        load_f32_chunk<IBF16, VEC>(irow, chunk[k], iv[k]);
        load_f32_chunk<IBF16, VEC>(grow, chunk[k], gv[k]);
      } else {
        p[k] = u32x4{0, 0, 0, 0};
#pragma unroll
        for (int e = 0; e < VEC; ++e) iv[k][e] = gv[k][e] = 0.f;
      }
    }

    float ss = 0.f, dt = 0.f, ga = 0.f;
#pragma unroll
    for (int k = 0; k < V; ++k) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float v = C::elem(p[k], e);
        ss = __builtin_fmaf(v, v, ss);
        dt = __builtin_fmaf(v, qw[k][e], dt);
        ga = __builtin_fmaf(gv[k][e], v - iv[k][e], ga);
      }
    }
    ss = wave_sum_to_lane63(ss);
    dt = wave_sum_to_lane63(dt);
    ga = wave_sum_to_lane63(ga);
    if (lane == 63) {
      red[ph][wave][0] = ss;
      red[ph][wave][1] = dt;
      red[ph][wave][2] = ga;
    }
    __syncthreads();
    float tss = 0.f, tdt = 0.f, tga = 0.f;
    for (int w = 0; w < nwaves; ++w) {
      tss += red[ph][w][0];
      tdt += red[ph][w][1];
      tga += red[ph][w][2];
    }
    ph ^= 1;
    const float r = __builtin_amdgcn_rsqf(tss * P.inv_d + P.eps);
    const float logit = tdt * r;
    // pi = sigmoid(z) and 1 - pi = sigmoid(-z), each from its own exponential:
    // as pi -> 1, 1.0 - pi (the reference's form, kernels/phase_2.py:141) or
    // G - pi G keeps none of the small values of 1 - pi below fp32's spacing
    // near 1, which dinter = (1 - pi) G and pi (1 - pi) need
    const float z = logit - P.inter_lse[tok];
    const float pi = 1.0f / (1.0f + __expf(-z));
    const float qi = 1.0f / (1.0f + __expf(z));
    const float gl = pi * qi * tga;
    if (tid == 0 && P.grad_lse) P.grad_lse[tok] = -gl;
    const float cq = uniform_f32(gl * r);
    const float cp = uniform_f32(-gl * logit * r * r * P.inv_d);
    const float pu = uniform_f32(pi);
    const float qu = uniform_f32(qi);

    char* gprow = reinterpret_cast<char*>(P.grad_partial) + tok * (int64_t)P.d * C::BYTES;
    char* girow = reinterpret_cast<char*>(P.grad_inter) + tok * (int64_t)P.d * IB;
    const __amdgpu_buffer_rsrc_t prs = row_rsrc(gprow, (uint32_t)(P.d * C::BYTES));
    const __amdgpu_buffer_rsrc_t irs = row_rsrc(girow, (uint32_t)(P.d * IB));
#pragma unroll
    for (int k = 0; k < V; ++k) {
      if (!ok[k]) continue;
      float dp[VEC], di[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float v = C::elem(p[k], e);
        dp[e] = __builtin_fmaf(cp, v, __builtin_fmaf(cq, qw[k][e], pu * gv[k][e]));
        di[e] = qu * gv[k][e];
        dqa[k][e] = __builtin_fmaf(cq, v, dqa[k][e]);
      }
      store_f32_chunk<PBF16, VEC>(prs, chunk[k], dp);
      store_f32_chunk<IBF16, VEC>(irs, chunk[k], di);
    }
  }

  float* qrow = P.dq_part + (int64_t)blockIdx.x * P.d;
#pragma unroll
  for (int k = 0; k < V; ++k) {
    if (!ok[k]) continue;
#pragma unroll
    for (int e = 0; e < VEC; ++e) qrow[(int64_t)chunk[k] * VEC + e] = dqa[k][e];
  }
}

// Stage 1 of the query-gradient reduction: workgroup (x, y) sums partial
// rows [64y, 64y+64) of columns [64x, 64x+64) in a fixed order (four waves of
// 16 rows, then the four wave sums in order) and stores the sum in row 64y,
// which no other workgroup reads or writes.
__device__ __forceinline__ void reduce_dqw_stage_body(const attnres_reduce_params& P) {
  __shared__ float red[4][64];
  const int lane = threadIdx.x & 63;
  const int slice = threadIdx.x >> 6;
  const int width = P.d * (P.num_queries > 1 ? P.num_queries : 1);
  const int col = blockIdx.x * 64 + lane;
  const int row0 = blockIdx.y * 64;
  float acc = 0.f;
  if (col < width) {
    const int r0 = row0 + slice * 16;
    const int r1 = r0 + 16 < P.nparts ? r0 + 16 : P.nparts;
#pragma unroll 16
    for (int r = r0; r < r1; ++r) acc += P.part[(int64_t)r * width + col];
  }
  red[slice][lane] = acc;
  __syncthreads();
  if (slice == 0 && col < width)
    P.part[(int64_t)row0 * width + col] = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
}

// The whole query-gradient reduction in one launch: workgroup x (1024
// threads) owns columns [32x, 32x + 32) of every query, so each wave reads
// whole 128-byte lines of two partial rows.  Thread (r, c) = (tid / 32,
// tid % 32) sums partial rows r, r + 32, r + 64, ... of column c in that
// order (32 rows of one query requested at once, through a buffer resource
// over the nparts rows with 32-bit offsets; rows past the end read zeros);
// the 32 row lanes are then added in a fixed tree through LDS (lanes
// 4k..4k+3 in order, then the 8 sums in order) and the fold
// qw = query * gain is applied backwards: dquery = dqw * gain, dgain = sum
// over queries (in order) of dqw * query.  Every sum has a fixed order, so
// the result is deterministic.
__device__ __forceinline__ void reduce_dqw_cols_body(const attnres_reduce_params& P) {
  constexpr int CW = 32, RL = 32, QB = 1, RB = 32;
  __shared__ float red[QB][RL][CW + 1];
  __shared__ float red2[QB][RL / 4][CW + 1];
  const int c = threadIdx.x & (CW - 1), r = threadIdx.x / CW;
  const int col = blockIdx.x * CW + c;
  const bool in = col < P.d;
  const int nq = P.num_queries > 1 ? P.num_queries : 1;
  const int64_t width = (int64_t)P.d * nq;
  const __amdgpu_buffer_rsrc_t rs = row_rsrc(reinterpret_cast<char*>(P.part), (uint32_t)(P.nparts * width * 4));
  float g = 1.f;
  if (P.gain && in) g = P.param_bf16 ? bf_lo(reinterpret_cast<const uint16_t*>(P.gain)[col])
                                     : reinterpret_cast<const float*>(P.gain)[col];
  float dg = 0.f;
  for (int q0 = 0; q0 < nq; q0 += QB) {
    float acc[QB];
#pragma unroll
    for (int b = 0; b < QB; ++b) acc[b] = 0.f;
    if (in) {
      // lane offsets carry the row (so rows at or past nparts fail the
      // resource's range check and read zeros), the scalar offset the query
      // column block within a row
      for (int r0 = r; r0 < P.nparts; r0 += RL * RB) {
        float v[QB][RB];
#pragma unroll
        for (int b = 0; b < QB; ++b) {
          const uint32_t soff = (uint32_t)((int64_t)(q0 + b) * P.d * 4);
#pragma unroll
          for (int j = 0; j < RB; ++j) {
            const uint32_t voff = (uint32_t)(((int64_t)(r0 + RL * j) * width + col) * 4);
            v[b][j] = q0 + b < nq ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, voff, soff, 0))
                                  : 0.f;
          }
        }
#pragma unroll
        for (int b = 0; b < QB; ++b) {
#pragma unroll
          for (int j = 0; j < RB; ++j) acc[b] += v[b][j];
        }
      }
    }
#pragma unroll
    for (int b = 0; b < QB; ++b) red[b][r][c] = acc[b];
    __syncthreads();
    if (r < RL / 4) {
#pragma unroll
      for (int b = 0; b < QB; ++b)
        red2[b][r][c] = ((red[b][4 * r][c] + red[b][4 * r + 1][c]) + red[b][4 * r + 2][c]) + red[b][4 * r + 3][c];
    }
    __syncthreads();
    if (r == 0 && in) {
#pragma unroll
      for (int b = 0; b < QB; ++b) {
        const int qi = q0 + b;
        if (qi >= nq) break;
        float t = 0.f;
#pragma unroll
        for (int k = 0; k < RL / 4; ++k) t += red2[b][k][c];
        const int64_t ci = (int64_t)qi * P.d + col;
        const float q = P.param_bf16 ? bf_lo(reinterpret_cast<const uint16_t*>(P.query)[ci])
                                     : reinterpret_cast<const float*>(P.query)[ci];
        const float dq = P.gain ? t * g : t;
        dg = __builtin_fmaf(t, q, dg);
        if (P.dquery) {
          if (P.param_bf16) reinterpret_cast<__bf16*>(P.dquery)[ci] = (__bf16)dq;
          else reinterpret_cast<float*>(P.dquery)[ci] = dq;
        }
      }
    }
    __syncthreads();
  }
  if (r == 0 && in && P.dgain) {
    if (P.param_bf16) reinterpret_cast<__bf16*>(P.dgain)[col] = (__bf16)dg;
    else reinterpret_cast<float*>(P.dgain)[col] = dg;
  }
}

// Final stage: sum the partial rows 0, part_step, 2*part_step, ... column by
// column (fixed order, so the result is deterministic) and apply the fold
// qw = query * gain backwards.
__device__ __forceinline__ void reduce_dqw_body(const attnres_reduce_params& P) {
  const int col = blockIdx.x * blockDim.x + threadIdx.x;
  if (col >= P.d) return;
  const int nq = P.num_queries > 1 ? P.num_queries : 1;
  const int64_t width = (int64_t)P.d * nq;
  const int nrows = (P.nparts + P.part_step - 1) / P.part_step;  // rows 0, part_step, 2 part_step, ...
  float g = 1.f;
  if (P.gain) g = P.param_bf16 ? bf_lo(reinterpret_cast<const uint16_t*>(P.gain)[col])
                               : reinterpret_cast<const float*>(P.gain)[col];
  float dg = 0.f;
  // QB queries x RB rows requested at once; each query's rows summed in row order
  constexpr int QB = 4, RB = 16;
  for (int q0 = 0; q0 < nq; q0 += QB) {
    float acc[QB];
#pragma unroll
    for (int b = 0; b < QB; ++b) acc[b] = 0.f;
    for (int r0 = 0; r0 < nrows; r0 += RB) {
      float v[QB][RB];
#pragma unroll
      for (int b = 0; b < QB; ++b) {
#pragma unroll
        for (int j = 0; j < RB; ++j) {
          const bool in = q0 + b < nq && r0 + j < nrows;
          v[b][j] = in ? P.part[(int64_t)(r0 + j) * P.part_step * width + (int64_t)(q0 + b) * P.d + col] : 0.f;
        }
      }
#pragma unroll
      for (int b = 0; b < QB; ++b) {
#pragma unroll
        for (int j = 0; j < RB; ++j) {
          if (r0 + j < nrows) acc[b] += v[b][j];
        }
      }
    }
#pragma unroll
    for (int b = 0; b < QB; ++b) {
      const int qi = q0 + b;
      if (qi >= nq) break;
      const int64_t c = (int64_t)qi * P.d + col;
      const float q = P.param_bf16 ? bf_lo(reinterpret_cast<const uint16_t*>(P.query)[c])
                                   : reinterpret_cast<const float*>(P.query)[c];
      const float dq = P.gain ? acc[b] * g : acc[b];
      dg = __builtin_fmaf(acc[b], q, dg);
      if (P.dquery) {
        if (P.param_bf16) reinterpret_cast<__bf16*>(P.dquery)[c] = (__bf16)dq;
        else reinterpret_cast<float*>(P.dquery)[c] = dq;
      }
    }
  }
  if (P.dgain) {
    if (P.param_bf16) reinterpret_cast<__bf16*>(P.dgain)[col] = (__bf16)dg;
    else reinterpret_cast<float*>(P.dgain)[col] = dg;
  }
}

}  // namespace

// ------------------------------------------------------- instantiations --
//
// Symbol names (looked up by the host launcher with hipModuleGetFunction):
//   attnres_route_<in>_<qw>_s<S>_v<V>_<q1|qn>
//     in : bf (bf16 sources) | f32 (fp32 sources)
//     qw : d2 (bf16-exact query, v_dot2 path) | fm (fp32 FMA path)
//   attnres_merge_<partial>_<inter>_v<V>

#define ROUTE_LB(V) __launch_bounds__(512)

#define ROUTE_ONE(INNAME, BF, QNAME, QD2, S, V)                                                        \
  extern "C" __global__ void ROUTE_LB(V) attnres_route_##INNAME##_##QNAME##_s##S##_v##V##_q1(         \
      attnres_route_params P) {                                                                       \
    route_body<S, V, BF, QD2, false>(P);                                                              \
  }                                                                                                   \
  extern "C" __global__ void ROUTE_LB(V) attnres_route_##INNAME##_##QNAME##_s##S##_v##V##_qn(         \
      attnres_route_params P) {                                                                       \
    route_body<S, V, BF, QD2, true>(P);                                                               \
  }

// bf16 sources and parameters, Q >= 2, bf16 output: the batched-query body
#define ROUTE_QG(S, V)                                                                                \
  extern "C" __global__ void ROUTE_LB(V) attnres_route_bf_d2_s##S##_v##V##_qg(attnres_route_params P) { \
    route_qg_body<S, V>(P);                                                                           \
  }
#define ROUTE_TYPES(S, V)                 \
  ROUTE_ONE(bf, true, d2, true, S, V)     \
  ROUTE_ONE(bf, true, fm, false, S, V)    \
  ROUTE_ONE(f32, false, fm, false, S, V)  \
  ROUTE_QG_IF(S, V)

#define ROUTE_QG_IF(S, V) ROUTE_QG_##S(V)
#define ROUTE_QG_0(V)
#define ROUTE_QG_1(V) ROUTE_QG(1, V)
#define ROUTE_QG_2(V) ROUTE_QG(2, V)
#define ROUTE_QG_3(V) ROUTE_QG(3, V)
#define ROUTE_QG_4(V) ROUTE_QG(4, V)
#define ROUTE_QG_5(V) ROUTE_QG(5, V)
#define ROUTE_QG_6(V) ROUTE_QG(6, V)
#define ROUTE_QG_7(V) ROUTE_QG(7, V)
#define ROUTE_QG_8(V) ROUTE_QG(8, V)
#define ROUTE_QG_9(V) ROUTE_QG(9, V)
#define ROUTE_QG_10(V) ROUTE_QG(10, V)
#define ROUTE_QG_11(V) ROUTE_QG(11, V)
#define ROUTE_QG_12(V) ROUTE_QG(12, V)
#define ROUTE_QG_13(V) ROUTE_QG(13, V)
#define ROUTE_QG_14(V) ROUTE_QG(14, V)
#define ROUTE_QG_15(V) ROUTE_QG(15, V)
#define ROUTE_QG_16(V) ROUTE_QG(16, V)
#define ROUTE_S(S) \
  ROUTE_TYPES(S, 1) \
  ROUTE_TYPES(S, 2)

// The build compiles this file once per module part (ATTNRES_PART = 0..10)
// so the parts build in parallel; the host maps each symbol to its part.
#ifndef ATTNRES_PART
#define ATTNRES_PART 0
#define ATTNRES_ALL_PARTS 1
#endif

#if ATTNRES_PART == 0 || defined(ATTNRES_ALL_PARTS)
ROUTE_S(0)
ROUTE_S(1)
ROUTE_S(2)
ROUTE_S(3)
ROUTE_S(4)
ROUTE_S(5)
#endif
#if ATTNRES_PART == 1 || defined(ATTNRES_ALL_PARTS)
ROUTE_S(6)
ROUTE_S(7)
ROUTE_S(8)
ROUTE_S(9)
#endif
#if ATTNRES_PART == 2 || defined(ATTNRES_ALL_PARTS)
ROUTE_S(10)
ROUTE_S(11)
ROUTE_S(12)
ROUTE_S(13)
#endif
#if ATTNRES_PART == 3 || defined(ATTNRES_ALL_PARTS)
ROUTE_S(14)
ROUTE_S(15)
ROUTE_S(16)

#define MERGE_ONE(PN, PB, IN, IB, V)                                                                 \
  extern "C" __global__ void ROUTE_LB(V) attnres_merge_##PN##_##IN##_v##V(attnres_merge_params P) { \
    merge_body<V, PB, IB>(P);                                                                        \
  }

#define MERGE_V(V)                   \
  MERGE_ONE(bf, true, bf, true, V)   \
  MERGE_ONE(bf, true, f32, false, V) \
  MERGE_ONE(f32, false, bf, true, V) \
  MERGE_ONE(f32, false, f32, false, V)

MERGE_V(1)
MERGE_V(2)
// Row-per-wave merge: attnres_merge_stream_<qw>_c<NCH> (bf16 rows of NCH KiB;
// qw: d2 = bf16 query on the v_dot2 path, fm = fp32 query), four waves per
// workgroup.
#define MERGE_STREAM(NCH)                                                                            \
  extern "C" __global__ void __launch_bounds__(256) attnres_merge_stream_d2_c##NCH(attnres_merge_params P) { \
    merge_stream_body<NCH, true>(P);                                                                 \
  }                                                                                                  \
  extern "C" __global__ void __launch_bounds__(256) attnres_merge_stream_fm_c##NCH(attnres_merge_params P) { \
    merge_stream_body<NCH, false>(P);                                                                \
  }
MERGE_STREAM(1)
MERGE_STREAM(2)
MERGE_STREAM(3)
MERGE_STREAM(4)
MERGE_STREAM(5)
MERGE_STREAM(6)
MERGE_STREAM(7)
MERGE_STREAM(8)
#endif

// Streaming kernels: attnres_stream_<in>_<qw>_c<NCH>_<plain|table|fused|fusedtable>, row = NCH KiB.
// Occupancy target (waves per SIMD): the plain and table kernels run one
// wave per SIMD (one workgroup per CU), so their register budget also holds
// the staged output rows past the LDS slots.
#define STREAM_WAVES_PER_EU(NCH) 1
// The fused kernels also hold the delta row of both pipeline slots.
#define STREAM_FUSED_WAVES_PER_EU(NCH) ((NCH) <= 3 ? 4 : (NCH) <= 4 ? 3 : 2)

#define STREAM_ONE_OUT(INNAME, BF, QNAME, QD2, ONAME, OBF, NCH)                                        \
  extern "C" __global__ void __launch_bounds__(64 * ATTNRES_STREAM_WAVES)                               \
      __attribute__((amdgpu_waves_per_eu(STREAM_WAVES_PER_EU(NCH))))                                    \
      attnres_stream_##INNAME##_##QNAME##_o##ONAME##_c##NCH##_plain(attnres_route_params P) {           \
    stream_body<NCH, BF, QD2, false, OBF, false>(P);                                                    \
  }                                                                                                     \
  extern "C" __global__ void __launch_bounds__(64 * ATTNRES_STREAM_WAVES)                               \
      __attribute__((amdgpu_waves_per_eu(STREAM_WAVES_PER_EU(NCH))))                                    \
      attnres_stream_##INNAME##_##QNAME##_o##ONAME##_c##NCH##_table(attnres_route_params P) {           \
    stream_body<NCH, BF, QD2, false, OBF, true>(P);                                                     \
  }                                                                                                     \
  extern "C" __global__ void __launch_bounds__(64 * ATTNRES_STREAM_WAVES)                               \
      __attribute__((amdgpu_waves_per_eu(STREAM_FUSED_WAVES_PER_EU(NCH))))                              \
      attnres_stream_##INNAME##_##QNAME##_o##ONAME##_c##NCH##_fused(attnres_route_params P) {           \
    stream_body<NCH, BF, QD2, true, OBF, false>(P);                                                     \
  }                                                                                                     \
  extern "C" __global__ void __launch_bounds__(64 * ATTNRES_STREAM_WAVES)                               \
      __attribute__((amdgpu_waves_per_eu(STREAM_FUSED_WAVES_PER_EU(NCH))))                              \
      attnres_stream_##INNAME##_##QNAME##_o##ONAME##_c##NCH##_fusedtable(attnres_route_params P) {      \
    stream_body<NCH, BF, QD2, true, OBF, true>(P);                                                      \
  }
#define STREAM_ONE(INNAME, BF, QNAME, QD2, NCH)             \
  STREAM_ONE_OUT(INNAME, BF, QNAME, QD2, bf, true, NCH)     \
  STREAM_ONE_OUT(INNAME, BF, QNAME, QD2, f32, false, NCH)

#define STREAM_TYPES(NCH)                 \
  STREAM_ONE(bf, true, d2, true, NCH)     \
  STREAM_ONE(bf, true, fm, false, NCH)    \
  STREAM_ONE(f32, false, fm, false, NCH)

#if ATTNRES_PART == 2 || defined(ATTNRES_ALL_PARTS)
STREAM_TYPES(1)
STREAM_TYPES(2)
STREAM_TYPES(3)
STREAM_TYPES(4)
#endif
#if ATTNRES_PART == 1 || defined(ATTNRES_ALL_PARTS)
STREAM_TYPES(5)
STREAM_TYPES(6)
STREAM_TYPES(7)
STREAM_TYPES(8)
#endif

// Backward: attnres_route_bwd_<in>_g<grad_out>_s<S>_v<V>; column reduce:
// attnres_reduce_dqw_cols (one launch, up to four queries) or
// attnres_reduce_dqw_stage + attnres_reduce_dqw (two).
// Waves per SIMD the backward kernels are compiled for: 4 (<= 128 VGPRs) keeps
// two workgroups of up to 8 waves (rows up to 4096 bf16 / 2048 fp32 elements)
// resident per CU for S <= 9; S = 9 bf16 spills a few dwords under that cap.
#ifndef ATTNRES_BWD_CAP_MAX_S
#define ATTNRES_BWD_CAP_MAX_S 9
#endif
#define BWD_WAVES_PER_EU(S, V) ((V) == 1 && (S) <= ATTNRES_BWD_CAP_MAX_S ? 4 : 1)
#define BWD_ONE(INNAME, BF, GNAME, GBF, S, V)                                                          \
  extern "C" __global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(BWD_WAVES_PER_EU(S, V)))) \
  attnres_route_bwd_##INNAME##_g##GNAME##_s##S##_v##V(attnres_route_bwd_params P) {                    \
    route_bwd_body<S, V, BF, GBF>(P);                                                                  \
  }
#define BWD_TYPES(S, V)                 \
  BWD_ONE(bf, true, bf, true, S, V)     \
  BWD_ONE(bf, true, f32, false, S, V)   \
  BWD_ONE(f32, false, f32, false, S, V) \
  BWD_ONE(f32, false, bf, true, S, V)
#define BWD_S(S)    \
  BWD_TYPES(S, 1) \
  BWD_TYPES(S, 2)

// Row-per-wave backward: attnres_route_bwd_stream_c<NCH>_s<S> (bf16 sources
// and output gradients, rows of NCH KiB).  Up to 48 / NCH source rows are
// kept in registers (S * NCH * 4 of them, partly in the accumulation
// registers); the 8 KiB instances with S = 7..9 keep their first KL = S - 6
// rows in LDS (KL * 8 KiB per wave).
#define BWD_STREAM_ONE(S, NCH, KL)                                                                      \
  extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1)))            \
      attnres_route_bwd_stream_c##NCH##_s##S(attnres_route_bwd_params P) {                               \
    route_bwd_stream_body<S, NCH, KL>(P);                                                               \
  }

#if ATTNRES_PART == 4 || defined(ATTNRES_ALL_PARTS)
BWD_STREAM_ONE(1, 6, 0) BWD_STREAM_ONE(2, 6, 0) BWD_STREAM_ONE(3, 6, 0) BWD_STREAM_ONE(4, 6, 0)
BWD_STREAM_ONE(5, 6, 0) BWD_STREAM_ONE(6, 6, 0) BWD_STREAM_ONE(7, 6, 0) BWD_STREAM_ONE(8, 6, 0)
BWD_STREAM_ONE(1, 8, 0) BWD_STREAM_ONE(2, 8, 0) BWD_STREAM_ONE(3, 8, 0) BWD_STREAM_ONE(4, 8, 0)
BWD_STREAM_ONE(5, 8, 0) BWD_STREAM_ONE(6, 8, 0) BWD_STREAM_ONE(7, 8, 1) BWD_STREAM_ONE(8, 8, 2)
BWD_STREAM_ONE(9, 8, 3)
BWD_S(1)
BWD_S(2)
BWD_S(3)
BWD_S(4)
BWD_S(5)
BWD_S(6)
BWD_S(7)
BWD_S(8)
// Merge backward: attnres_merge_bwd_<partial>_<inter>_v<V>.
#define MERGE_BWD_ONE(PN, PB, IN, IB, V)                                                             \
  extern "C" __global__ void __launch_bounds__(512) attnres_merge_bwd_##PN##_##IN##_v##V(             \
      attnres_merge_bwd_params P) {                                                                  \
    merge_bwd_body<V, PB, IB>(P);                                                                    \
  }
#define MERGE_BWD_V(V)                   \
  MERGE_BWD_ONE(bf, true, bf, true, V)   \
  MERGE_BWD_ONE(bf, true, f32, false, V) \
  MERGE_BWD_ONE(f32, false, bf, true, V) \
  MERGE_BWD_ONE(f32, false, f32, false, V)
MERGE_BWD_V(1)
MERGE_BWD_V(2)
extern "C" __global__ void __launch_bounds__(256) attnres_reduce_dqw_stage(attnres_reduce_params P) {
  reduce_dqw_stage_body(P);
}
extern "C" __global__ void __launch_bounds__(256) attnres_reduce_dqw(attnres_reduce_params P) { reduce_dqw_body(P); }
extern "C" __global__ void __launch_bounds__(1024) attnres_reduce_dqw_cols(attnres_reduce_params P) {
  reduce_dqw_cols_body(P);
}
#endif
#if ATTNRES_PART == 5 || defined(ATTNRES_ALL_PARTS)
BWD_S(9)
BWD_S(10)
BWD_S(11)
BWD_S(12)
BWD_S(13)
BWD_S(14)
BWD_S(15)
BWD_S(16)
#endif

// Batched-query backward: attnres_route_bwd_mq_<in>_g<grad_out>_s<S>_v<V>,
// instantiated where the per-thread source-gradient accumulators (S * VEC * V
// floats) stay within 72 registers; attnres_route_bwd_dqw_<in>_v<V>.
#define BWD_MQ_ONE(INNAME, BF, GNAME, GBF, S, V)                                                  \
  extern "C" __global__ void __launch_bounds__(512)                                               \
  attnres_route_bwd_mq_##INNAME##_g##GNAME##_s##S##_v##V(attnres_route_bwd_mq_params P) {       \
    route_bwd_mq_body<S, V, BF, GBF>(P);                                                          \
  }
#define BWD_MQ(INNAME, BF, S, V) \
  BWD_MQ_ONE(INNAME, BF, bf, true, S, V) \
  BWD_MQ_ONE(INNAME, BF, f32, false, S, V)
#define BWD_DQW(INNAME, BF, V)                                                                   \
  extern "C" __global__ void __launch_bounds__(512)                                              \
  attnres_route_bwd_dqw_##INNAME##_v##V(attnres_route_bwd_dqw_params P) {                        \
    route_bwd_dqw_body<V, BF>(P);                                                                \
  }
#if ATTNRES_PART == 6 || defined(ATTNRES_ALL_PARTS)
BWD_MQ(bf, true, 1, 1) BWD_MQ(bf, true, 2, 1) BWD_MQ(bf, true, 3, 1) BWD_MQ(bf, true, 4, 1) BWD_MQ(bf, true, 5, 1)
BWD_MQ(bf, true, 6, 1) BWD_MQ(bf, true, 7, 1) BWD_MQ(bf, true, 8, 1) BWD_MQ(bf, true, 9, 1)
BWD_MQ(bf, true, 1, 2) BWD_MQ(bf, true, 2, 2) BWD_MQ(bf, true, 3, 2) BWD_MQ(bf, true, 4, 2)
BWD_MQ(f32, false, 1, 1) BWD_MQ(f32, false, 2, 1) BWD_MQ(f32, false, 3, 1) BWD_MQ(f32, false, 4, 1)
BWD_MQ(f32, false, 5, 1) BWD_MQ(f32, false, 6, 1) BWD_MQ(f32, false, 7, 1) BWD_MQ(f32, false, 8, 1)
BWD_MQ(f32, false, 9, 1) BWD_MQ(f32, false, 10, 1) BWD_MQ(f32, false, 11, 1) BWD_MQ(f32, false, 12, 1)
BWD_MQ(f32, false, 13, 1) BWD_MQ(f32, false, 14, 1) BWD_MQ(f32, false, 15, 1) BWD_MQ(f32, false, 16, 1)
BWD_MQ(f32, false, 1, 2) BWD_MQ(f32, false, 2, 2) BWD_MQ(f32, false, 3, 2) BWD_MQ(f32, false, 4, 2)
BWD_MQ(f32, false, 5, 2) BWD_MQ(f32, false, 6, 2) BWD_MQ(f32, false, 7, 2) BWD_MQ(f32, false, 8, 2)
BWD_MQ(f32, false, 9, 2)
BWD_DQW(bf, true, 1) BWD_DQW(bf, true, 2) BWD_DQW(f32, false, 1) BWD_DQW(f32, false, 2)
#endif

// Batched-query backward on the matrix cores (bf16 sources, output gradients
// and parameters): attnres_route_bwd_mqg_s<S>_q<NQ4>, up to 4*NQ4 queries, two
// chunks per thread, at most 256 threads (rows of up to 4096 bf16 elements).
#ifndef MQG_WAVES_PER_EU
#define MQG_WAVES_PER_EU(S, NQ4) 2
#endif
#define BWD_MQG(S, NQ4)                                                                         \
  extern "C" __global__ void __launch_bounds__(256)                                             \
      __attribute__((amdgpu_waves_per_eu(MQG_WAVES_PER_EU(S, NQ4))))                            \
      attnres_route_bwd_mqg_s##S##_q##NQ4(attnres_route_bwd_mq_params P) {                      \
    route_bwd_mqg_body<S, 2, NQ4>(P);                                                           \
  }
#define BWD_DQWM(V)                                                                             \
  extern "C" __global__ void __launch_bounds__(512) attnres_route_bwd_dqwm_bf_v##V(             \
      attnres_route_bwd_dqw_params P) {                                                         \
    route_bwd_dqwm_body<V>(P);                                                                  \
  }
#if ATTNRES_PART == 7 || defined(ATTNRES_ALL_PARTS)
BWD_DQWM(1) BWD_DQWM(2)
BWD_MQG(1, 1) BWD_MQG(2, 1) BWD_MQG(3, 1) BWD_MQG(4, 1) BWD_MQG(5, 1) BWD_MQG(6, 1) BWD_MQG(7, 1) BWD_MQG(8, 1)
BWD_MQG(1, 2) BWD_MQG(2, 2) BWD_MQG(3, 2) BWD_MQG(4, 2) BWD_MQG(5, 2) BWD_MQG(6, 2) BWD_MQG(7, 2) BWD_MQG(8, 2)
#endif

// Backward with addend rows (dsrc[s] = dx_s + dadd[s]; in place when dadd[s] is
// dsrc[s]): attnres_route_bwd_<in>_g<grad_out>_s<S>_v<V>_add for bf16 sources
// with bf16 output gradients and fp32 with fp32, and
// attnres_route_bwd_stream_c<NCH>_s<S>_add.  The same register targets as
// the kernels without addends.
#define BWD_ONE_ADD(INNAME, BF, GNAME, GBF, S, V)                                                      \
  extern "C" __global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(BWD_WAVES_PER_EU(S, V)))) \
  attnres_route_bwd_##INNAME##_g##GNAME##_s##S##_v##V##_add(attnres_route_bwd_params P) {              \
    route_bwd_body<S, V, BF, GBF, true>(P);                                                            \
  }
#define BWD_S_ADD(S)                          \
  BWD_ONE_ADD(bf, true, bf, true, S, 1)       \
  BWD_ONE_ADD(bf, true, bf, true, S, 2)       \
  BWD_ONE_ADD(f32, false, f32, false, S, 1)   \
  BWD_ONE_ADD(f32, false, f32, false, S, 2)
#define BWD_STREAM_ONE_ADD(S, NCH, KL)                                                                  \
  extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1)))            \
      attnres_route_bwd_stream_c##NCH##_s##S##_add(attnres_route_bwd_params P) {                         \
    route_bwd_stream_body<S, NCH, KL, true>(P);                                                         \
  }

#if ATTNRES_PART == 8 || defined(ATTNRES_ALL_PARTS)
BWD_STREAM_ONE_ADD(1, 6, 0) BWD_STREAM_ONE_ADD(2, 6, 0) BWD_STREAM_ONE_ADD(3, 6, 0) BWD_STREAM_ONE_ADD(4, 6, 0)
BWD_STREAM_ONE_ADD(5, 6, 0) BWD_STREAM_ONE_ADD(6, 6, 0) BWD_STREAM_ONE_ADD(7, 6, 0) BWD_STREAM_ONE_ADD(8, 6, 0)
BWD_STREAM_ONE_ADD(1, 8, 0) BWD_STREAM_ONE_ADD(2, 8, 0) BWD_STREAM_ONE_ADD(3, 8, 0) BWD_STREAM_ONE_ADD(4, 8, 0)
BWD_STREAM_ONE_ADD(5, 8, 0) BWD_STREAM_ONE_ADD(6, 8, 0) BWD_STREAM_ONE_ADD(7, 8, 1) BWD_STREAM_ONE_ADD(8, 8, 2)
BWD_STREAM_ONE_ADD(9, 8, 3)
BWD_S_ADD(1)
BWD_S_ADD(2)
BWD_S_ADD(3)
BWD_S_ADD(4)
#endif
#if ATTNRES_PART == 9 || defined(ATTNRES_ALL_PARTS)
BWD_S_ADD(5)
BWD_S_ADD(6)
BWD_S_ADD(7)
BWD_S_ADD(8)
BWD_S_ADD(9)
BWD_S_ADD(10)
BWD_S_ADD(11)
BWD_S_ADD(12)
BWD_S_ADD(13)
BWD_S_ADD(14)
BWD_S_ADD(15)
BWD_S_ADD(16)
#endif

// Deferred block gradients (the training loop's routing points):
// attnres_route_bwd_stream_c<NCH>_s<S>_defer, the row-per-wave backward that
// forms only the last source's gradient and stores the committed sources'
// coefficients (summed by the segment kernels below).
#define BWD_STREAM_ONE_DEFER(S, NCH, KL)                                                                \
  extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1)))            \
      attnres_route_bwd_stream_c##NCH##_s##S##_defer(attnres_route_bwd_params P) {                       \
    route_bwd_stream_body<S, NCH, KL, true, true>(P);                                                   \
  }

#if ATTNRES_PART == 10 || defined(ATTNRES_ALL_PARTS)
BWD_STREAM_ONE_DEFER(2, 6, 0) BWD_STREAM_ONE_DEFER(3, 6, 0) BWD_STREAM_ONE_DEFER(4, 6, 0)
BWD_STREAM_ONE_DEFER(5, 6, 0) BWD_STREAM_ONE_DEFER(6, 6, 0) BWD_STREAM_ONE_DEFER(7, 6, 0)
BWD_STREAM_ONE_DEFER(8, 6, 0)
BWD_STREAM_ONE_DEFER(2, 8, 0) BWD_STREAM_ONE_DEFER(3, 8, 0) BWD_STREAM_ONE_DEFER(4, 8, 0)
BWD_STREAM_ONE_DEFER(5, 8, 0) BWD_STREAM_ONE_DEFER(6, 8, 0) BWD_STREAM_ONE_DEFER(7, 8, 1)
BWD_STREAM_ONE_DEFER(8, 8, 2) BWD_STREAM_ONE_DEFER(9, 8, 3)
BWD_STREAM_ONE_DEFER(2, 2, 0) BWD_STREAM_ONE_DEFER(3, 2, 0) BWD_STREAM_ONE_DEFER(4, 2, 0)
BWD_STREAM_ONE_DEFER(5, 2, 0) BWD_STREAM_ONE_DEFER(6, 2, 0) BWD_STREAM_ONE_DEFER(7, 2, 0)
BWD_STREAM_ONE_DEFER(8, 2, 0)
BWD_STREAM_ONE_DEFER(2, 1, 0) BWD_STREAM_ONE_DEFER(3, 1, 0) BWD_STREAM_ONE_DEFER(4, 1, 0)
BWD_STREAM_ONE_DEFER(5, 1, 0) BWD_STREAM_ONE_DEFER(6, 1, 0) BWD_STREAM_ONE_DEFER(7, 1, 0)
BWD_STREAM_ONE_DEFER(8, 1, 0)
#endif

// Segments of deferred sums (the instances in ATTNRES_SEG_INSTANCES), a wave
// per CPW KiB part of a row with a ring of DEPTH items, compiled for WPE
// waves per SIMD.  Measured at the 3B and 8B shapes (8 terms, 32768 and 16384
// rows): the kernels are bound by their loads and stores, not the matrix
// cores (removing the MFMAs or the A operands' construction changed nothing,
// removing the stores took 15-30% off); larger parts read faster, so up to
// four blocks (one group, 32 fp32 sums per KiB and lane) take 3 KiB (6 KiB
// rows) or 4 KiB parts (8 KiB rows), five to eight blocks (two groups) 2 KiB
// parts with a shallow ring, where 1 KiB parts ran 5-8% slower at 6 KiB
// rows.  Non-temporal stores beat sc1 and default ones by 5-15%.
#define GATHER_SEG_ONE(NCH, NB, CPW, DEPTH, WPE)                                                        \
  extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE)))          \
      attnres_route_bwd_gather_seg_c##NCH##_b##NB(attnres_route_bwd_gather_seg_params P) {              \
    route_bwd_gather_seg_body<NB, NCH, CPW, DEPTH>(P);                                                  \
  }
#if ATTNRES_PART == 10 || defined(ATTNRES_ALL_PARTS)
ATTNRES_SEG_INSTANCES(GATHER_SEG_ONE)
#endif
