// Shared device helpers for the gfx950 (MI355X) speculative-decoding kernels.
//
// Storage type for bf16 is uint16_t everywhere (bit patterns); arithmetic is fp32.
// Rounding fp32 -> bf16 is round-to-nearest-even, the same rule torch uses.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ssd_mi355x.h"

#define SSD_API extern "C" __attribute__((visibility("default")))

typedef uint16_t bf16_t;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;

namespace ssd {

// Host-side error reporting: every entry point returns 0 on success, else a
// nonzero code and a message retrievable through ssd_last_error().
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
// Counts every kernel the library enqueues (read with ssd_launch_count); SSD_LAUNCH is
// hipLaunchKernelGGL plus the count.
void count_launch();
#define SSD_LAUNCH(...)          \
  do {                           \
    ::ssd::count_launch();       \
    hipLaunchKernelGGL(__VA_ARGS__); \
  } while (0)

enum Status {
  SSD_OK = 0,
  SSD_EINVAL = 1,     // bad argument (shape, pointer, size)
  SSD_ERANGE = 2,     // size beyond a compiled limit
  SSD_EHIP = 3,       // HIP runtime error
};

__device__ __forceinline__ float bf2f(bf16_t v) { return __uint_as_float(((uint32_t)v) << 16); }

typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2_t;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;

// Two fp32 -> packed bf16 pair (lo in bits 0-15): one v_cvt_pk_bf16_f32 on gfx950 (round to
// nearest even, NaN stays NaN).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ bf16_t f2bf(float f) { return (bf16_t)(pack_bf16x2(f, 0.f) & 0xffffu); }

// Round through bf16 (the value an fp32 result takes once stored as bf16).
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

union Pack8 {
  uint4 u;
  bf16_t h[8];
  bf16x8_t v;
};

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 u) {
  Pack8 p;
  p.u = u;
  return p.v;
}

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// Reinterpret 8 packed bf16 (four 32-bit words) as the MFMA operand type (no memory round trip).
__device__ __forceinline__ bf16x8_t bits_bf16x8(u32x4_t u) { return __builtin_bit_cast(bf16x8_t, u); }

// Streaming (non-temporal) 16-byte load: weights are read once per call, keep them out of the caches' way.
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
  const u32x4_t v = __builtin_nontemporal_load((const u32x4_t*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// ---- KV-cache layout: 64-slot blocks stored as the attention kernel's MFMA operands.
// One (layer, kv head) holds max_len slots (a multiple of 64) of K and of V, max_len * hd
// elements each. Slot s sits in block s / 64 at offset o = s % 64.
//  K: block b is 4 * hd/32 operand tiles (kt, ks) of 64 lanes x 8 bf16, tile (kt, ks) lane
//     (g * 16 + i) = K[slot 64b + key(kt, i)][32 ks + 8 g .. + 8], key(kt, i) =
//     (kt / 2) * 32 + (i / 4) * 8 + (kt % 2) * 4 + i % 4: the A operand of S^T = K Q^T for key
//     tile kt and k-step ks, so the attention kernel loads each tile as one contiguous 1 KiB.
//  V: block b is hd/16 x 2 tiles (dt, c), tile (dt, c) lane (g * 16 + i) = V[slots 64b + 32c +
//     8g .. + 8][dim 16 dt + i]: the A operand of O^T = V^T P^T for dim tile dt and key half c.
__device__ __forceinline__ int kv_key_tile(int o) { return ((o >> 5) << 1) | ((o >> 2) & 1); }
__device__ __forceinline__ int kv_key_lane(int o) { return (((o >> 3) & 3) << 2) | (o & 3); }
// element offset of K[s][d] (d and the 8 following dims of the same 8-group are contiguous)
__device__ __forceinline__ size_t k_off(int s, int d, int hd) {
  const int o = s & 63;
  return ((((size_t)(s >> 6) * 4 + kv_key_tile(o)) * (hd >> 5) + (d >> 5)) * 64 + ((d >> 3) & 3) * 16 +
          kv_key_lane(o)) * 8 + (d & 7);
}
// element offset of V[s][d] (slots s .. s + 7 of the same 8-group are contiguous)
__device__ __forceinline__ size_t v_off(int s, int d, int hd) {
  const int o = s & 63;
  return ((((size_t)(s >> 6) * (hd >> 4) + (d >> 4)) * 2 + (o >> 5)) * 64 + ((o >> 3) & 3) * 16 + (d & 15)) * 8 +
         (o & 7);
}

__device__ __forceinline__ f32x4_t mfma16x16x32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }
__device__ __forceinline__ float gelu_f(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f)); }
__device__ __forceinline__ float relu_f(float x) { return x > 0.f ? x : 0.f; }

// Entry points with per-row KV arena offsets (element offset of each row's sequence, or null), for
// forwards whose rows belong to several sequences (batched generation); the exported
// ssd_gemm_qkv_rope_bf16 / ssd_tree_attention_bf16 are these with null offsets.
int qkv_rope_gemm(const uint16_t* X, int64_t ldx, int M, const uint16_t* W_packed, int K, float norm_eps, int heads,
                  int kv_heads, int head_dim, const uint16_t* cos_tab, const uint16_t* sin_tab, int64_t rope_rows,
                  const int32_t* row_pos, const int32_t* row_slot, const int64_t* row_kv_off, uint16_t* Q,
                  int64_t ldq, uint16_t* k_cache, uint16_t* vt_cache, int64_t max_len, hipStream_t stream);
int tree_attention(const uint16_t* q, int64_t ldq, int M, int heads, int kv_heads, int head_dim,
                   const uint16_t* k_cache, const uint16_t* vt_cache, int64_t max_len, const int32_t* prefix,
                   const int32_t* depth, const int32_t* anc, const int64_t* kv_off, int p_min, int l_max, float scale,
                   float* ws, int64_t ws_floats, uint16_t* out, int64_t ldo, hipStream_t stream);

enum Act { ACT_NONE = 0, ACT_SILU = 1, ACT_GELU = 2, ACT_RELU = 3 };

__device__ __forceinline__ float apply_act(int act, float x) {
  switch (act) {
    case ACT_SILU: return silu_f(x);
    case ACT_GELU: return gelu_f(x);
    case ACT_RELU: return relu_f(x);
    default: return x;
  }
}

// Device-scope (agent) loads and stores: how workgroups of one launch hand data to each other
// across CUs and XCDs (a plain store may sit in the writer's L2; a plain load may hit a line the
// reader's L2 cached earlier in the launch).
__device__ __forceinline__ uint32_t ld_agent_u32(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent_u32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent_u64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until every global load and store this wave issued has completed; also a compiler barrier
// (no memory access moves across it).
__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

}  // namespace ssd
