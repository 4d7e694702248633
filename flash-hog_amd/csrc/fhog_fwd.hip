// Flash attention forward on gfx950: O = softmax(scale Q K^T) V and the
// natural-log row logsumexp L, the residual the first and second backward
// consume. Replaces the cuDNN forward that the reference calls through
// flash_hog/jax/_attention_impl.py:224-239 (L is (batch, heads, tokens) fp32,
// natural log, of the scaled and masked logits).
//
// A workgroup owns 128 queries (4 waves x 32) of one (batch, head) and streams
// 32-key tiles of K and V through LDS. Scores are computed transposed
// (S^T = K Q^T) and the output as O^T = V^T P^T, so every lane holds one query
// row in both: the online-softmax rescale is a per-lane scalar multiply.
#include "fhog_device.h"
#include "fhog_params.h"

namespace fhog {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;

template <typename T, int D, bool CAUSAL>
__global__ void __launch_bounds__(kThreads) fwd_kernel(FwdParams<T> p) {
  typedef TileGeom<T, D> G;
  constexpr int KS = D / 16;
  constexpr int DT = D / 32;
  constexpr int BQ = 32 * kWaves;
  constexpr int BK = 32;
  __shared__ __attribute__((aligned(32))) T s_row[2][2][G::kRowElems];  // K, V
  __shared__ __attribute__((aligned(32))) T s_tr[2][2][G::kTrElems];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 31, g = lane >> 5;
  const int nqb = (p.nq + BQ - 1) / BQ;
  const int lin = xcd_remap(blockIdx.x, nqb * p.batch * p.heads);
  const int bh = lin / nqb;
  const int qb = CAUSAL ? nqb - 1 - lin % nqb : lin % nqb;
  const int b = bh / p.heads, h = bh % p.heads;
  const long rs = (long)p.heads * D;
  const long qbase = ((long)b * p.nq * p.heads + h) * D;
  const long kbase = ((long)b * p.nk * p.heads + h) * D;
  const long sbase = (long)bh * p.nq;
  const int q0 = qb * BQ + wave * 32;
  const int qi = q0 + n;
  const bool qvalid = qi < p.nq;

  V8<T> qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const long off = qbase + (long)qi * rs + 16 * ks + 8 * g;
    qf[ks] = qvalid ? *reinterpret_cast<const V8<T>*>(p.q + off) : zero8<T>();
  }

  int kend = p.nk;
  if (CAUSAL) kend = min(kend, qb * BQ + BQ);
  const int nkt = (kend + BK - 1) / BK;
  int wend = p.nk;
  if (CAUSAL) wend = min(wend, q0 + 32);
  const int wkt = q0 < p.nq ? (wend + BK - 1) / BK : 0;

  const float c2 = p.scale * kLog2e;
  float m = -1e30f;  // running row max of the log2-domain logits
  float lpart = 0.f; // this lane's share of the running row sum
  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = zero16();

  const bool loader = wave < 2;
  const T* src = (wave == 0 ? p.k : p.v) + kbase;
  TileRegs<T, D> pre;
  if (loader) {
    tile_load<T, D>(pre, src, rs, p.nk, lane);
    tile_store_lds<T, D>(pre, s_row[0][wave], s_tr[0][wave], lane);
  }
  __syncthreads();

  for (int kt = 0; kt < nkt; ++kt) {
    const int buf = kt & 1;
    const bool has_next = kt + 1 < nkt;
    if (has_next && loader) tile_load<T, D>(pre, src + (long)(kt + 1) * BK * rs, rs, p.nk - (kt + 1) * BK, lane);
    if (kt < wkt) {
      const T* sK = s_row[buf][0];
      f32x16 S = zero16();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) S = mma<T>(frag_row<T, D>(sK, n, g, ks), qf[ks], S);
      const int k0 = kt * BK;
      const bool need_mask = (k0 + BK > p.nk) || (CAUSAL && k0 + BK - 1 > q0);
      float mloc = -1e30f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float s2 = S[r] * c2;
        if (need_mask) {
          const int kj = k0 + crow(r, g);
          const bool ok = kj < p.nk && (!CAUSAL || kj <= qi);
          s2 = ok ? s2 : -INFINITY;
        }
        S[r] = s2;
        mloc = fmaxf(mloc, s2);
      }
      const float mnew = fmaxf(m, xgroup_max(mloc));
      const float alpha = exp2_fast(m - mnew);
      m = mnew;
      float psum = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pv = exp2_fast(S[r] - mnew);  // masked: exp2(-inf) = 0
        S[r] = pv;
        psum += pv;
      }
      lpart = lpart * alpha + psum;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc[dt] *= alpha;
      const T* tV = s_tr[buf][1];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const V8<T> oP = cvt8<T>(s ? hi8(S) : lo8(S));
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[dt] = mma<T>(frag_tr<T, D>(tV, 32 * dt + n, g, s), oP, acc[dt]);
      }
    }
    if (has_next && loader) tile_store_lds<T, D>(pre, s_row[buf ^ 1][wave], s_tr[buf ^ 1][wave], lane);
    __syncthreads();
  }

  const float l = xgroup_sum(lpart);
  if (qvalid) {
    const float inv = 1.f / l;
    T* o = p.o + qbase + (long)qi * rs;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        f32x4 x;
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = acc[dt][4 * a + j] * inv;
        *reinterpret_cast<V4<T>*>(o + 32 * dt + 8 * a + 4 * g) = cvt4<T>(x);
      }
    }
    if (g == 0) p.lse[sbase + qi] = (m + __log2f(l)) * kLn2;
  }
}

}  // namespace

template <typename T, int D, bool CAUSAL>
hipError_t launch_fwd(const FwdParams<T>& p, hipStream_t stream) {
  const int nqb = (p.nq + 32 * kWaves - 1) / (32 * kWaves);
  hipLaunchKernelGGL((fwd_kernel<T, D, CAUSAL>), dim3(nqb * p.batch * p.heads), dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

#define FHOG_INST(T, D, C) template hipError_t launch_fwd<T, D, C>(const FwdParams<T>&, hipStream_t);
FHOG_INST(__bf16, 64, true)
FHOG_INST(__bf16, 64, false)
FHOG_INST(__bf16, 128, true)
FHOG_INST(__bf16, 128, false)
FHOG_INST(_Float16, 64, true)
FHOG_INST(_Float16, 64, false)
FHOG_INST(_Float16, 128, true)
FHOG_INST(_Float16, 128, false)
FHOG_INST(float, 64, true)
FHOG_INST(float, 64, false)
#undef FHOG_INST

}  // namespace fhog
