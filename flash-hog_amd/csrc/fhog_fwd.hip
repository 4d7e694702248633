// Flash attention forward on gfx950: O = softmax(scale Q K^T) V and the
// natural-log row logsumexp L, the residual the first and second backward
// consume. Replaces the cuDNN forward that the reference calls through
// flash_hog/jax/_attention_impl.py:224-239 (L is (batch, heads, tokens) fp32,
// natural log, of the scaled and masked logits).
//
// A workgroup owns 128 queries (4 waves x 32) of one (batch, head) and streams
// 32-key tiles of K and V global -> LDS (no registers) through a 4-stage ring
// of XOR-swizzled tiles, one barrier per tile; wave w loads half (w % 2) of
// tensor w / 2. Scores are computed transposed (S^T = K Q^T) and the output
// as O^T = V^T P^T, so every lane holds one query row in both: the online-
// softmax rescale is a per-lane scalar multiply, skipped when no row of the
// wave raised its running maximum. Causal blocks are issued longest first with
// (batch, head) as the minor index (see fhog_bwdbwd.hip).
#include "fhog_device.h"
#include "fhog_params.h"

namespace fhog {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kStages = 4;  // 3 stages: 0.5-1 % slower

// Waves per SIMD the register allocator is asked to allow: three for 2-byte
// types at D = 64 (119 VGPRs; 50.7 against 55.4 us at two waves, B4 N2048 H16
// causal, and four waves are no faster), two at D = 128 (190 VGPRs, no spill;
// 147.7 against 86.3 us at one wave, B4 N2048 H16 causal) and for fp32 at
// D = 64 (154 VGPRs; 167 against 154 us at B2 N2048 H8), one otherwise.
template <typename T, int D> struct Occupancy {
  static constexpr int value = sizeof(T) != 2 ? (D == 64 ? 2 : 1) : D == 64 ? 3 : D == 128 ? 2 : 1;
};

template <typename T, int D, bool CAUSAL>
__global__ void __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(Occupancy<T, D>::value, Occupancy<T, D>::value)))
fwd_kernel(FwdParams<T> p, int chunk) {
  typedef SwzTile<T, D> G;
  constexpr int KS = D / 16;
  constexpr int DT = D / 32;
  constexpr int BQ = 32 * kWaves;
  constexpr int BK = 32;
  constexpr int NST = kStages;
  constexpr int kTile = G::kElems * (int)sizeof(T);
  constexpr int kStage = 2 * kTile;  // K, V
  constexpr int kPer = G::kLoads / 2;
  __shared__ __attribute__((aligned(1024))) char s_kv[NST * kStage];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 31, g = lane >> 5;
  const int nqb = (p.nq + BQ - 1) / BQ;
  const int nbh = p.batch * p.heads;
  const GridSlot gs = grid_slot(blockIdx.x, nbh, nqb, chunk);
  const int bh = gs.pair;
  const int qb = CAUSAL ? nqb - 1 - gs.rank : gs.rank;  // causal: the longest query rows first
  const int b = bh / p.heads, h = bh % p.heads;
  const int hk = h / (p.heads / p.kv_heads);
  const long rs = (long)p.heads * D;      // query-side row stride
  const long rsk = (long)p.kv_heads * D;  // key-side row stride
  const long qbase = ((long)b * p.nq * p.heads + h) * D;
  const long kbase = ((long)b * p.nk * p.kv_heads + hk) * D;
  const long sbase = (long)bh * p.nq;
  const int q0 = qb * BQ + wave * 32;
  const int qi = q0 + n;
  const bool qvalid = qi < p.nq;

  // A negative scale is applied as |scale| to -Q (negation is exact), so the
  // logits the running maximum is taken over are the unscaled scores of -Q.
  const bool negate = p.scale < 0.f;
  V8<T> qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const long off = qbase + (long)qi * rs + 16 * ks + 8 * g;
    qf[ks] = qvalid ? *reinterpret_cast<const V8<T>*>(p.q + off) : zero8<T>();
    if (negate) qf[ks] = -qf[ks];
  }

  // Keys [0, kend) are visible to some query of the workgroup, [0, wend) to
  // some query of this wave.
  int kend = p.nk;
  if (CAUSAL) kend = min(kend, qb * BQ + BQ + p.coff);
  // (uniform; saying so keeps the compiler from treating the loop as divergent)
  const int nkt = __builtin_amdgcn_readfirstlane(kend > 0 ? (kend + BK - 1) / BK : 0);
  int wend = p.nk;
  if (CAUSAL) wend = max(0, min(wend, q0 + 32 + p.coff));
  const int wkt = q0 < p.nq ? (wend + BK - 1) / BK : 0;

  SwzFrags<T, D> fr;
  fr.init(lane);
  const int tensor = wave >> 1;  // 0 = K, 1 = V
  const T* src = (tensor == 0 ? p.k : p.v) + kbase;
  const uint32_t row_bytes = (uint32_t)(rsk * (long)sizeof(T));
  TileDma<T, D, kPer> dma;
  dma.init(row_bytes, BK, lane, kPer * (wave & 1));
  const uint32_t lds_kv = lds_base_u32(s_kv);
  const uint32_t lds_tensor = lds_kv + tensor * kTile;
  auto issue = [&](int kt) {
    const int nvalid = p.nk - kt * BK;
    const uint32_t dst = lds_tensor + (uint32_t)(((uint32_t)kt % NST) * kStage);
    const T* gsrc = src + (long)kt * BK * rsk;
    if (nvalid >= BK) {
      dma.issue(dst, gsrc);
    } else {
      TileDma<T, D, kPer> part;
      part.init(row_bytes, nvalid, lane, kPer * (wave & 1));
      part.issue(dst, gsrc);
    }
  };

  const float c2 = fabsf(p.scale) * kLog2e;  // > 0
  constexpr float kBound = 256.f;  // bound on P (2^8)
  float m = -1e30f;  // running row max of the log2-domain logits (possibly stale, see below)
  float lpart = 0.f; // this lane's share of the running row sum
  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = zero16();

  // Retire the query loads before the ring starts: otherwise the compiler waits
  // for them at their first use inside the loop, and that wait (vmcnt counts
  // the untracked LDS DMAs too) would drain the prefetched tiles.
  wait_vmem();
#pragma unroll
  for (int i = 0; i < NST - 1; ++i)
    if (i < nkt) issue(i);

  for (int kt = 0; kt < nkt; ++kt) {
    wait_tile<NST, kPer>(kt, nkt);
    __syncthreads();
    if (kt + NST - 1 < nkt) issue(kt + NST - 1);
    if (kt < wkt) {
      const uint32_t sa = lds_kv + (uint32_t)(((uint32_t)kt % NST) * kStage);  // K at 0, V at kTile
      f32x16 S = zero16();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) S = mma<T>(fr.rowf(sa, 0, ks), qf[ks], S);
      // S stays unscaled: the row maximum is taken on it and scaled once
      // (c2 > 0, and rounding is monotonic, so this equals the maximum of the
      // scaled values), and the scale enters the exponent's fma below.
      const int k0 = kt * BK;
      if ((k0 + BK > p.nk) || (CAUSAL && k0 + BK - 1 > q0 + p.coff)) {
        const int klim = min(p.nk - 1, CAUSAL ? qi + p.coff : p.nk - 1) - k0;  // last visible key, tile-relative
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (crow(r, g) > klim) S[r] = -INFINITY;
      }
      // Lazy rescale: a row keeps its running maximum m (log2 units) while the
      // probabilities it gives stay small, and O, l carry the same stale factor,
      // which the final O / l and L = m + log2 l cancel. P is formed with the
      // stale m first. If a lane's 16 values sum to more than kBound, or
      // overflow (the first tile, with m = -1e30, always does), the wave takes
      // the row maximum, rescales O and l to it and forms P again; so
      // P <= kBound. Most tiles thus skip the maximum (15 max and a cross-lane
      // exchange) and the rescale (an exp and 33 multiplies).
      f32x16 P;
      float psum = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        P[r] = exp2_fast(fmaf(S[r], c2, -m));  // masked: exp2(-inf) = 0
        psum += P[r];
      }
      if (__any(!(psum <= kBound))) {
        float mloc = S[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mloc = fmaxf(mloc, S[r]);
        const float mnew = fmaxf(m, xgroup_max(mloc * c2));
        const float alpha = exp2_fast(m - mnew);
        lpart *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[dt] *= alpha;
        m = mnew;
        psum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          P[r] = exp2_fast(fmaf(S[r], c2, -m));
          psum += P[r];
        }
      }
      lpart += psum;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const V8<T> oP = cvt8<T>(s ? hi8(P) : lo8(P));
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[dt] = mma<T>(fr.trf(sa, kTile, dt, s), oP, acc[dt]);
      }
    }
  }

  // A query that sees no key (bottom-right causal with nq > nk) gets O = 0 and
  // L = +inf, so that every backward kernel computes P = exp(S - L) = 0 for it.
  const float l = xgroup_sum(lpart);
  if (qvalid) {
    const float inv = l > 0.f ? 1.f / l : 0.f;
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
    if (g == 0) p.lse[sbase + qi] = l > 0.f ? (m + __log2f(l)) * kLn2 : INFINITY;
  }
}

}  // namespace

template <typename T, int D, bool CAUSAL>
hipError_t launch_fwd(const FwdParams<T>& p, hipStream_t stream) {
  const int nqb = (p.nq + 32 * kWaves - 1) / (32 * kWaves);
  const int npairs = p.batch * p.heads;
  const int chunk = grid_chunk(npairs, nqb, resident_workgroups(Occupancy<T, D>::value));
  hipLaunchKernelGGL((fwd_kernel<T, D, CAUSAL>), dim3(nqb * npairs), dim3(kThreads), 0, stream, p, chunk);
  return hipGetLastError();
}

#define FHOG_INST(T, D, C) template hipError_t launch_fwd<T, D, C>(const FwdParams<T>&, hipStream_t);
FHOG_INST(__bf16, 64, true)
FHOG_INST(__bf16, 64, false)
FHOG_INST(__bf16, 128, true)
FHOG_INST(__bf16, 128, false)
FHOG_INST(__bf16, 256, true)
FHOG_INST(__bf16, 256, false)
FHOG_INST(_Float16, 64, true)
FHOG_INST(_Float16, 64, false)
FHOG_INST(_Float16, 128, true)
FHOG_INST(_Float16, 128, false)
FHOG_INST(_Float16, 256, true)
FHOG_INST(_Float16, 256, false)
FHOG_INST(float, 64, true)
FHOG_INST(float, 64, false)
FHOG_INST(float, 128, true)
FHOG_INST(float, 128, false)
#undef FHOG_INST

}  // namespace fhog
