// Flash-HOG double backward of softmax attention on gfx950: two kernels, no
// atomics, no (N_Q, N_K) tensor.
//
// Per (batch, head), with S = scale Q K^T (causal: key > query masked),
// P = exp(S - L), dP = dO V^T, ddS = scale (ddQ K^T + Q ddK^T), dPa = dO ddV^T:
//   D  = rowsum(O * dO)                                  (fused into stage 1)
//   dD = rowsum(ddS * P)                                  pass 1
//   B  = rowsum(dP2 * P),  dP2 = dPa - dP dD - ddS D + dP ddS      pass 2
//   dQ2 = dS ddK + dS2 K,  ddO = P ddV + ddP V            pass 3
//   dK2 = dS^T ddQ + dS2^T Q,  dV2 = ddP^T dO             pass 4
// with dS = scale P (dP - D), dS2 = scale P (dP2 - B), ddP = P (ddS - dD).
// The math follows flash_hog/_jax_refs/jax_impl.py:273-336 and the pass split of
// flash_hog/jax/_pallas_gpu_kernel.py:149-391. Passes 1 and 2 share one sweep
// over the keys: B = r1 - dD r2 - D dD + r3 with r1 = rowsum(dPa P),
// r2 = rowsum(dP P), r3 = rowsum(dP ddS P), which is rowsum(dP2 P) expanded.
//
// Stage 1 (passes 1-3): a workgroup owns 128 queries (4 waves x 32) of one
// (batch, head) and streams 32-key tiles of K, V, ddK, ddV through LDS twice.
// Score tiles are computed transposed (S^T = K Q^T) so each lane holds one
// query row: row statistics are per-lane scalars and row sums need one
// cross-group add at the end of the sweep. The query-side operands stay in
// registers for the whole sweep.
//
// Stage 2 (pass 4): a workgroup owns 128 keys (4 waves x 32) and streams
// 32-query tiles of Q, dO, ddQ plus their row statistics through LDS. Score
// tiles are S = Q K^T, so each lane holds one key column.
#include "fhog_device.h"
#include "fhog_params.h"

namespace fhog {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;

// ----------------------------------------------------------------------------
// Stage 1: passes 1-3, tiled over queries.
// ----------------------------------------------------------------------------
template <typename T, int D, bool CAUSAL>
__global__ void __launch_bounds__(kThreads) bwdbwd_q_kernel(BwdBwdParams<T> p) {
  typedef TileGeom<T, D> G;
  constexpr int KS = D / 16;       // 16-deep steps over the head dim
  constexpr int DT = D / 32;       // 32-wide output column blocks
  constexpr int BQ = 32 * kWaves;  // queries per workgroup
  constexpr int BK = 32;           // keys per streamed tile
  // tensors: 0 = K, 1 = V, 2 = ddK, 3 = ddV
  __shared__ __attribute__((aligned(32))) T s_row[2][4][G::kRowElems];
  __shared__ __attribute__((aligned(32))) T s_tr[2][4][G::kTrElems];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 31, g = lane >> 5;
  const int nqb = (p.nq + BQ - 1) / BQ;
  const int lin = xcd_remap(blockIdx.x, nqb * p.batch * p.heads);
  const int bh = lin / nqb;
  const int qb = CAUSAL ? nqb - 1 - lin % nqb : lin % nqb;  // longest rows first
  const int b = bh / p.heads, h = bh % p.heads;
  const long rs = (long)p.heads * D;
  const long qbase = ((long)b * p.nq * p.heads + h) * D;
  const long kbase = ((long)b * p.nk * p.heads + h) * D;
  const long sbase = (long)bh * p.nq;
  const int q0 = qb * BQ + wave * 32;
  const int qi = q0 + n;
  const bool qvalid = qi < p.nq;

  // Query-side operands (B of the score products) and D_i = <O_i, dO_i>.
  V8<T> qf[KS], ddqf[KS], dof[KS];
  float dpart = 0.f;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const long off = qbase + (long)qi * rs + 16 * ks + 8 * g;
    if (qvalid) {
      qf[ks] = *reinterpret_cast<const V8<T>*>(p.q + off);
      ddqf[ks] = *reinterpret_cast<const V8<T>*>(p.ddq + off);
      dof[ks] = *reinterpret_cast<const V8<T>*>(p.dout + off);
      const V8<T> of = *reinterpret_cast<const V8<T>*>(p.o + off);
#pragma unroll
      for (int e = 0; e < 8; ++e) dpart += (float)of[e] * (float)dof[ks][e];
    } else {
      qf[ks] = zero8<T>();
      ddqf[ks] = zero8<T>();
      dof[ks] = zero8<T>();
    }
  }
  const float Di = xgroup_sum(dpart);
  const float Li2 = qvalid ? p.lse[sbase + qi] * kLog2e : 0.f;

  int kend = p.nk;
  if (CAUSAL) kend = min(kend, qb * BQ + BQ);
  const int nkt = (kend + BK - 1) / BK;           // tiles the workgroup streams
  int wend = p.nk;
  if (CAUSAL) wend = min(wend, q0 + 32);
  const int wkt = q0 < p.nq ? (wend + BK - 1) / BK : 0;  // tiles with work for this wave

  const float scale = p.scale;
  const float c2 = scale * kLog2e;
  float dd_acc = 0.f, r1 = 0.f, r2 = 0.f, r3 = 0.f;
  float ddi = 0.f, bi = 0.f;
  f32x16 acc_dq2[DT], acc_ddo[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    acc_dq2[dt] = zero16();
    acc_ddo[dt] = zero16();
  }

  const T* src = wave == 0 ? p.k : wave == 1 ? p.v : wave == 2 ? p.ddk : p.ddv;
  src += kbase;
  TileRegs<T, D> pre;
  tile_load<T, D>(pre, src, rs, p.nk, lane);
  tile_store_lds<T, D>(pre, s_row[0][wave], s_tr[0][wave], lane);
  __syncthreads();

  for (int it = 0; it < 2 * nkt; ++it) {
    const int kt = it < nkt ? it : it - nkt;
    const int buf = it & 1;
    const bool has_next = it + 1 < 2 * nkt;
    if (has_next) {
      const int ktn = it + 1 < nkt ? it + 1 : it + 1 - nkt;
      tile_load<T, D>(pre, src + (long)ktn * BK * rs, rs, p.nk - ktn * BK, lane);
    }
    if (kt < wkt) {
      const T* sK = s_row[buf][0];
      const T* sV = s_row[buf][1];
      const T* sdK = s_row[buf][2];
      const T* sdV = s_row[buf][3];
      f32x16 S = zero16(), ddS = zero16(), dP = zero16(), dPa = zero16();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const V8<T> kf = frag_row<T, D>(sK, n, g, ks);
        const V8<T> dkf = frag_row<T, D>(sdK, n, g, ks);
        const V8<T> vf = frag_row<T, D>(sV, n, g, ks);
        const V8<T> dvf = frag_row<T, D>(sdV, n, g, ks);
        S = mma<T>(kf, qf[ks], S);
        ddS = mma<T>(kf, ddqf[ks], ddS);
        ddS = mma<T>(dkf, qf[ks], ddS);
        dP = mma<T>(vf, dof[ks], dP);
        dPa = mma<T>(dvf, dof[ks], dPa);
      }
      const int k0 = kt * BK;
      const bool need_mask = (k0 + BK > p.nk) || (CAUSAL && k0 + BK - 1 > q0);
      f32x16 P;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float pv = exp2_fast(S[r] * c2 - Li2);
        if (need_mask) {
          const int kj = k0 + crow(r, g);
          const bool ok = kj < p.nk && (!CAUSAL || kj <= qi);
          pv = ok ? pv : 0.f;
        }
        P[r] = pv;
      }
      if (it < nkt) {
        // passes 1+2: per-lane partial row sums
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float pd = P[r] * dP[r];
          dd_acc += ddS[r] * P[r];
          r1 += dPa[r] * P[r];
          r2 += pd;
          r3 += pd * ddS[r];
        }
      } else {
        // pass 3
        f32x16 vdS, vdS2, vddP;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float ddss = ddS[r] * scale;
          const float t = ddss - ddi;
          const float dp = dP[r];
          const float dp2 = dPa[r] + dp * t - ddss * Di;
          const float ps = P[r] * scale;
          vdS[r] = ps * (dp - Di);
          vdS2[r] = ps * (dp2 - bi);
          vddP[r] = P[r] * t;
        }
        const T* tK = s_tr[buf][0];
        const T* tV = s_tr[buf][1];
        const T* tdK = s_tr[buf][2];
        const T* tdV = s_tr[buf][3];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const V8<T> oS = cvt8<T>(s ? hi8(vdS) : lo8(vdS));
          const V8<T> oS2 = cvt8<T>(s ? hi8(vdS2) : lo8(vdS2));
          const V8<T> odP = cvt8<T>(s ? hi8(vddP) : lo8(vddP));
          const V8<T> oP = cvt8<T>(s ? hi8(P) : lo8(P));
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            const int col = 32 * dt + n;
            acc_dq2[dt] = mma<T>(frag_tr<T, D>(tdK, col, g, s), oS, acc_dq2[dt]);
            acc_dq2[dt] = mma<T>(frag_tr<T, D>(tK, col, g, s), oS2, acc_dq2[dt]);
            acc_ddo[dt] = mma<T>(frag_tr<T, D>(tV, col, g, s), odP, acc_ddo[dt]);
            acc_ddo[dt] = mma<T>(frag_tr<T, D>(tdV, col, g, s), oP, acc_ddo[dt]);
          }
        }
      }
    }
    if (it == nkt - 1) {
      ddi = xgroup_sum(dd_acc) * scale;
      const float R1 = xgroup_sum(r1);
      const float R2 = xgroup_sum(r2);
      const float R3 = xgroup_sum(r3) * scale;
      bi = R1 - ddi * R2 - Di * ddi + R3;
    }
    if (has_next) tile_store_lds<T, D>(pre, s_row[buf ^ 1][wave], s_tr[buf ^ 1][wave], lane);
    __syncthreads();
  }

  if (qvalid) {
    T* dq2 = p.dq2 + qbase + (long)qi * rs;
    T* ddo = p.ddo + qbase + (long)qi * rs;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d = 32 * dt + 8 * a + 4 * g;
        f32x4 x, y;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          x[j] = acc_dq2[dt][4 * a + j];
          y[j] = acc_ddo[dt][4 * a + j];
        }
        *reinterpret_cast<V4<T>*>(dq2 + d) = cvt4<T>(x);
        *reinterpret_cast<V4<T>*>(ddo + d) = cvt4<T>(y);
      }
    }
    if (g == 0) {
      p.delta[sbase + qi] = Di;
      p.ddelta[sbase + qi] = ddi;
      p.bstat[sbase + qi] = bi;
    }
  }
}

// ----------------------------------------------------------------------------
// Stage 2: pass 4, tiled over keys.
// ----------------------------------------------------------------------------
template <typename T, int D, bool CAUSAL>
__global__ void __launch_bounds__(kThreads) bwdbwd_k_kernel(BwdBwdParams<T> p) {
  typedef TileGeom<T, D> G;
  constexpr int KS = D / 16;
  constexpr int DT = D / 32;
  constexpr int BKB = 32 * kWaves;  // keys per workgroup
  constexpr int BQ = 32;            // queries per streamed tile
  // tensors: 0 = Q, 1 = dO, 2 = ddQ; statistics: 0 = L log2(e), 1 = D, 2 = dD, 3 = B
  __shared__ __attribute__((aligned(32))) T s_row[2][3][G::kRowElems];
  __shared__ __attribute__((aligned(32))) T s_tr[2][3][G::kTrElems];
  __shared__ __attribute__((aligned(16))) float s_stat[2][4][BQ];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 31, g = lane >> 5;
  const int nkb = (p.nk + BKB - 1) / BKB;
  const int lin = xcd_remap(blockIdx.x, nkb * p.batch * p.heads);
  const int bh = lin / nkb;
  const int kb = lin % nkb;  // causal: the longest key columns come first
  const int b = bh / p.heads, h = bh % p.heads;
  const long rs = (long)p.heads * D;
  const long qbase = ((long)b * p.nq * p.heads + h) * D;
  const long kbase = ((long)b * p.nk * p.heads + h) * D;
  const long sbase = (long)bh * p.nq;
  const int k0 = kb * BKB + wave * 32;
  const int kj = k0 + n;
  const bool kvalid = kj < p.nk;

  const int nqt = (p.nq + BQ - 1) / BQ;
  const int qt_begin = CAUSAL ? (kb * BKB) / BQ : 0;

  f32x16 acc_dk2[DT], acc_dv2[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    acc_dk2[dt] = zero16();
    acc_dv2[dt] = zero16();
  }

  if (qt_begin < nqt) {
    // Key-side operands (B of the score products).
    V8<T> kf[KS], dkf[KS], vf[KS], dvf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const long off = kbase + (long)kj * rs + 16 * ks + 8 * g;
      if (kvalid) {
        kf[ks] = *reinterpret_cast<const V8<T>*>(p.k + off);
        dkf[ks] = *reinterpret_cast<const V8<T>*>(p.ddk + off);
        vf[ks] = *reinterpret_cast<const V8<T>*>(p.v + off);
        dvf[ks] = *reinterpret_cast<const V8<T>*>(p.ddv + off);
      } else {
        kf[ks] = zero8<T>();
        dkf[ks] = zero8<T>();
        vf[ks] = zero8<T>();
        dvf[ks] = zero8<T>();
      }
    }
    const float scale = p.scale;
    const float c2 = scale * kLog2e;

    const T* src = wave == 0 ? p.q : wave == 1 ? p.dout : p.ddq;
    src += qbase;
    TileRegs<T, D> pre;
    float2 st_pre;
    // statistics loader: wave 3, lane -> (statistic lane/16, queries 2(lane%16) + {0,1})
    const int st_id = lane >> 4, st_q = 2 * (lane & 15);
    const float* st_src = st_id == 0 ? p.lse : st_id == 1 ? p.delta : st_id == 2 ? p.ddelta : p.bstat;
    st_src += sbase;
    const float st_mul = st_id == 0 ? kLog2e : 1.f;

    auto load_tile = [&](int qt) {
      const int q0 = qt * BQ;
      if (wave < 3) {
        tile_load<T, D>(pre, src + (long)q0 * rs, rs, p.nq - q0, lane);
      } else {
        const int qa = q0 + st_q;
        st_pre.x = qa < p.nq ? st_src[qa] * st_mul : 0.f;
        st_pre.y = qa + 1 < p.nq ? st_src[qa + 1] * st_mul : 0.f;
      }
    };
    auto store_tile = [&](int buf) {
      if (wave < 3) {
        tile_store_lds<T, D>(pre, s_row[buf][wave], s_tr[buf][wave], lane);
      } else {
        *reinterpret_cast<float2*>(&s_stat[buf][st_id][st_q]) = st_pre;
      }
    };

    load_tile(qt_begin);
    store_tile(0);
    __syncthreads();

    for (int qt = qt_begin; qt < nqt; ++qt) {
      const int buf = (qt - qt_begin) & 1;
      const bool has_next = qt + 1 < nqt;
      if (has_next) load_tile(qt + 1);
      const int q0 = qt * BQ;
      const bool active = k0 < p.nk && (!CAUSAL || q0 + BQ - 1 >= k0);
      if (active) {
        const T* sQ = s_row[buf][0];
        const T* sdO = s_row[buf][1];
        const T* sdQ = s_row[buf][2];
        f32x16 S = zero16(), ddS = zero16(), dP = zero16(), dPa = zero16();
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const V8<T> qa = frag_row<T, D>(sQ, n, g, ks);
          const V8<T> dqa = frag_row<T, D>(sdQ, n, g, ks);
          const V8<T> doa = frag_row<T, D>(sdO, n, g, ks);
          S = mma<T>(qa, kf[ks], S);
          ddS = mma<T>(dqa, kf[ks], ddS);
          ddS = mma<T>(qa, dkf[ks], ddS);
          dP = mma<T>(doa, vf[ks], dP);
          dPa = mma<T>(doa, dvf[ks], dPa);
        }
        const bool need_mask = (q0 + BQ > p.nq) || (CAUSAL && q0 < k0 + 31);
        f32x16 vdS, vdS2, vddP;
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const int m0 = 8 * a + 4 * g;
          const f32x4 l2 = *reinterpret_cast<const f32x4*>(&s_stat[buf][0][m0]);
          const f32x4 dv = *reinterpret_cast<const f32x4*>(&s_stat[buf][1][m0]);
          const f32x4 ddv = *reinterpret_cast<const f32x4*>(&s_stat[buf][2][m0]);
          const f32x4 bv = *reinterpret_cast<const f32x4*>(&s_stat[buf][3][m0]);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int r = 4 * a + j;
            float pv = exp2_fast(S[r] * c2 - l2[j]);
            if (need_mask) {
              const int qg = q0 + m0 + j;
              const bool ok = qg < p.nq && (!CAUSAL || qg >= kj);
              pv = ok ? pv : 0.f;
            }
            const float ddss = ddS[r] * scale;
            const float t = ddss - ddv[j];
            const float dp = dP[r];
            const float dp2 = dPa[r] + dp * t - ddss * dv[j];
            const float ps = pv * scale;
            vdS[r] = ps * (dp - dv[j]);
            vdS2[r] = ps * (dp2 - bv[j]);
            vddP[r] = pv * t;
          }
        }
        const T* tQ = s_tr[buf][0];
        const T* tdO = s_tr[buf][1];
        const T* tdQ = s_tr[buf][2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const V8<T> oS = cvt8<T>(s ? hi8(vdS) : lo8(vdS));
          const V8<T> oS2 = cvt8<T>(s ? hi8(vdS2) : lo8(vdS2));
          const V8<T> odP = cvt8<T>(s ? hi8(vddP) : lo8(vddP));
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            const int col = 32 * dt + n;
            acc_dk2[dt] = mma<T>(frag_tr<T, D>(tdQ, col, g, s), oS, acc_dk2[dt]);
            acc_dk2[dt] = mma<T>(frag_tr<T, D>(tQ, col, g, s), oS2, acc_dk2[dt]);
            acc_dv2[dt] = mma<T>(frag_tr<T, D>(tdO, col, g, s), odP, acc_dv2[dt]);
          }
        }
      }
      if (has_next) store_tile(buf ^ 1);
      __syncthreads();
    }
  }

  if (kvalid) {
    T* dk2 = p.dk2 + kbase + (long)kj * rs;
    T* dv2 = p.dv2 + kbase + (long)kj * rs;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d = 32 * dt + 8 * a + 4 * g;
        f32x4 x, y;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          x[j] = acc_dk2[dt][4 * a + j];
          y[j] = acc_dv2[dt][4 * a + j];
        }
        *reinterpret_cast<V4<T>*>(dk2 + d) = cvt4<T>(x);
        *reinterpret_cast<V4<T>*>(dv2 + d) = cvt4<T>(y);
      }
    }
  }
}

}  // namespace

template <typename T, int D, bool CAUSAL>
hipError_t launch_bwdbwd(const BwdBwdParams<T>& p, hipStream_t stream, int stages) {
  const int nbh = p.batch * p.heads;
  const int nqb = (p.nq + 32 * kWaves - 1) / (32 * kWaves);
  const int nkb = (p.nk + 32 * kWaves - 1) / (32 * kWaves);
  if (stages & 1) {
    hipLaunchKernelGGL((bwdbwd_q_kernel<T, D, CAUSAL>), dim3(nqb * nbh), dim3(kThreads), 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (stages & 2) {
    hipLaunchKernelGGL((bwdbwd_k_kernel<T, D, CAUSAL>), dim3(nkb * nbh), dim3(kThreads), 0, stream, p);
    return hipGetLastError();
  }
  return hipSuccess;
}

#define FHOG_INST(T, D, C) template hipError_t launch_bwdbwd<T, D, C>(const BwdBwdParams<T>&, hipStream_t, int);
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
