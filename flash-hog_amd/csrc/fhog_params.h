// Launch parameter blocks and launcher declarations shared by the kernel files
// and the C-ABI translation unit.
//
// Tensors are BTNH (batch, tokens, heads, head_dim) and contiguous, the layout
// of the reference's attention seam; row statistics are (batch, heads, tokens)
// fp32, the layout of the reference's logsumexp residual.
//
// heads counts query heads (q, o, dout, ddq, dq, dq2, ddo and the row
// statistics); kv_heads counts key/value heads (k, v, ddk, ddv, dk, dv, dk2,
// dv2). Query head h reads key/value head h / (heads / kv_heads), the grouping
// of flash_hog/jax/_pallas_gpu_kernel.py:106-107 ("(kv_heads group)").
// Causal kernels show key j to query i iff j <= i + coff: coff = 0 aligns the
// mask top-left (_pallas_gpu_kernel.py:37-41), coff = nk - nq bottom-right
// (flash_hog/_jax_refs/jax_impl.py:104-109).
#pragma once

#include <hip/hip_runtime.h>

namespace fhog {

template <typename T> struct FwdParams {
  const T* q; const T* k; const T* v;
  T* o; float* lse;
  int batch, nq, nk, heads, kv_heads, coff;
  float scale;
};

template <typename T> struct BwdParams {
  const T* q; const T* k; const T* v; const T* o; const T* dout;
  const float* lse;
  T* dq; T* dk; T* dv;
  float* delta;
  int batch, nq, nk, heads, kv_heads, coff;
  float scale;
};

template <typename T> struct BwdBwdParams {
  const T* q; const T* k; const T* v; const T* o; const T* dout;
  const T* ddq; const T* ddk; const T* ddv;
  const float* lse;
  T* dq2; T* dk2; T* dv2; T* ddo;
  float* delta; float* ddelta; float* bstat;
  int batch, nq, nk, heads, kv_heads, coff;
  float scale;
};

// First query row whose pair with key kj enters dK2 and dV2. A query that
// sees no key but kj has a constant softmax (P = 1 whatever Q, K, V), so the
// pair's terms dS, dS2, ddP are exactly zero, while their fp32 forms cancel
// only to the rounding of the row statistics (about 1e-7 of |D dD| + |B|).
// Stage 2 drops such pairs as it drops masked ones: every row when nk = 1,
// else, under the causal mask, row -coff for key 0; rows before
// kj - coff do not see kj at all.
template <typename T>
__device__ inline int first_contributing_query(const BwdBwdParams<T>& p, int kj, bool causal) {
  if (p.nk == 1) return p.nq;
  return causal ? kj - p.coff + (kj == 0) : 0;
}

template <typename T, int D, bool CAUSAL> hipError_t launch_fwd(const FwdParams<T>& p, hipStream_t s);
template <typename T, int D, bool CAUSAL> hipError_t launch_bwd(const BwdParams<T>& p, hipStream_t s);
// stages: bit 0 = stage 1 (passes 1-3), bit 1 = stage 2 (pass 4).
template <typename T, int D, bool CAUSAL>
hipError_t launch_bwdbwd(const BwdBwdParams<T>& p, hipStream_t s, int stages = 3);
// Stage 1 in one sweep (2-byte types, D = 64 and 128); launch_bwdbwd selects it.
template <typename T, int D, bool CAUSAL>
hipError_t launch_bwdbwd_stage1_fused(const BwdBwdParams<T>& p, hipStream_t s);
// Stage 1 with 32 queries per wave at one wave per SIMD (2-byte types, D = 64);
// launch_bwdbwd selects it.
template <typename T, bool CAUSAL>
hipError_t launch_bwdbwd_stage1_q32(const BwdBwdParams<T>& p, hipStream_t s);
// Stage 2 with 32 keys per wave at one wave per SIMD (bf16, D = 64);
// launch_bwdbwd selects it.
template <bool CAUSAL>
hipError_t launch_bwdbwd_stage2_k32(const BwdBwdParams<__bf16>& p, hipStream_t s);
// The first backward's dK/dV kernel with 64 keys per wave at one wave per SIMD
// (2-byte types, D = 64); launch_bwd selects it for grids of whole rounds.
template <typename T, bool CAUSAL>
hipError_t launch_bwd_k64(const BwdParams<T>& p, hipStream_t s);
// The first backward's dQ kernel with 64 queries per wave at one wave per SIMD
// (2-byte types, D = 64); launch_bwd selects it for grids of whole rounds.
template <typename T, bool CAUSAL>
hipError_t launch_bwd_q64(const BwdParams<T>& p, hipStream_t s);
// Stage 2 with 16 keys per wave (2-byte types, D = 128); launch_bwdbwd selects it.
template <typename T, int D, bool CAUSAL>
hipError_t launch_bwdbwd_stage2_k16(const BwdBwdParams<T>& p, hipStream_t s);

}  // namespace fhog
