// First-order attention backward on gfx950, atomic free:
//   D  = rowsum(O * dO),  P = exp(scale Q K^T - L),  dP = dO V^T,
//   dS = scale P (dP - D),  dQ = dS K,  dK = dS^T Q,  dV = P^T dO.
// Replaces the cuDNN backward that the reference calls through
// flash_hog/jax/_attention_impl.py:242-261; the equations are those of
// flash_hog/_jax_refs/jax_impl.py:142-191 (attn_bwd).
//
// Kernel 1 (tiled over queries) computes D for its rows, writes it, and
// accumulates dQ while streaming K and V. Kernel 2 (tiled over keys) reads D
// and accumulates dK and dV while streaming Q, dO and the row statistics.
// Score tiles use the same transposed-versus-direct orientation as the
// double backward so that every row statistic is a per-lane scalar or a
// 4-wide LDS read.
#include "fhog_device.h"
#include "fhog_params.h"

namespace fhog {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;

template <typename T, int D, bool CAUSAL>
__global__ void __launch_bounds__(kThreads) bwd_q_kernel(BwdParams<T> p) {
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

  V8<T> qf[KS], dof[KS];
  float dpart = 0.f;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const long off = qbase + (long)qi * rs + 16 * ks + 8 * g;
    if (qvalid) {
      qf[ks] = *reinterpret_cast<const V8<T>*>(p.q + off);
      dof[ks] = *reinterpret_cast<const V8<T>*>(p.dout + off);
      const V8<T> of = *reinterpret_cast<const V8<T>*>(p.o + off);
#pragma unroll
      for (int e = 0; e < 8; ++e) dpart += (float)of[e] * (float)dof[ks][e];
    } else {
      qf[ks] = zero8<T>();
      dof[ks] = zero8<T>();
    }
  }
  const float Di = xgroup_sum(dpart);
  const float Li2 = qvalid ? p.lse[sbase + qi] * kLog2e : 0.f;

  int kend = p.nk;
  if (CAUSAL) kend = min(kend, qb * BQ + BQ);
  const int nkt = (kend + BK - 1) / BK;
  int wend = p.nk;
  if (CAUSAL) wend = min(wend, q0 + 32);
  const int wkt = q0 < p.nq ? (wend + BK - 1) / BK : 0;

  const float scale = p.scale;
  const float c2 = scale * kLog2e;
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
      const T* sV = s_row[buf][1];
      f32x16 S = zero16(), dP = zero16();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        S = mma<T>(frag_row<T, D>(sK, n, g, ks), qf[ks], S);
        dP = mma<T>(frag_row<T, D>(sV, n, g, ks), dof[ks], dP);
      }
      const int k0 = kt * BK;
      const bool need_mask = (k0 + BK > p.nk) || (CAUSAL && k0 + BK - 1 > q0);
      f32x16 vdS;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float pv = exp2_fast(S[r] * c2 - Li2);
        if (need_mask) {
          const int kj = k0 + crow(r, g);
          const bool ok = kj < p.nk && (!CAUSAL || kj <= qi);
          pv = ok ? pv : 0.f;
        }
        vdS[r] = pv * scale * (dP[r] - Di);
      }
      const T* tK = s_tr[buf][0];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const V8<T> oS = cvt8<T>(s ? hi8(vdS) : lo8(vdS));
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[dt] = mma<T>(frag_tr<T, D>(tK, 32 * dt + n, g, s), oS, acc[dt]);
      }
    }
    if (has_next && loader) tile_store_lds<T, D>(pre, s_row[buf ^ 1][wave], s_tr[buf ^ 1][wave], lane);
    __syncthreads();
  }

  if (qvalid) {
    T* dq = p.dq + qbase + (long)qi * rs;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        f32x4 x;
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = acc[dt][4 * a + j];
        *reinterpret_cast<V4<T>*>(dq + 32 * dt + 8 * a + 4 * g) = cvt4<T>(x);
      }
    }
    if (g == 0) p.delta[sbase + qi] = Di;
  }
}

template <typename T, int D, bool CAUSAL>
__global__ void __launch_bounds__(kThreads) bwd_k_kernel(BwdParams<T> p) {
  typedef TileGeom<T, D> G;
  constexpr int KS = D / 16;
  constexpr int DT = D / 32;
  constexpr int BKB = 32 * kWaves;
  constexpr int BQ = 32;
  // tensors: 0 = Q, 1 = dO; statistics: 0 = L log2(e), 1 = D
  __shared__ __attribute__((aligned(32))) T s_row[2][2][G::kRowElems];
  __shared__ __attribute__((aligned(32))) T s_tr[2][2][G::kTrElems];
  __shared__ __attribute__((aligned(16))) float s_stat[2][2][BQ];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 31, g = lane >> 5;
  const int nkb = (p.nk + BKB - 1) / BKB;
  const int lin = xcd_remap(blockIdx.x, nkb * p.batch * p.heads);
  const int bh = lin / nkb;
  const int kb = lin % nkb;
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

  f32x16 acc_dk[DT], acc_dv[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    acc_dk[dt] = zero16();
    acc_dv[dt] = zero16();
  }

  if (qt_begin < nqt) {
    V8<T> kf[KS], vf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const long off = kbase + (long)kj * rs + 16 * ks + 8 * g;
      kf[ks] = kvalid ? *reinterpret_cast<const V8<T>*>(p.k + off) : zero8<T>();
      vf[ks] = kvalid ? *reinterpret_cast<const V8<T>*>(p.v + off) : zero8<T>();
    }
    const float scale = p.scale;
    const float c2 = scale * kLog2e;

    const T* src = (wave == 0 ? p.q : p.dout) + qbase;
    TileRegs<T, D> pre;
    float st_pre = 0.f;
    // statistics loader: wave 2, lane -> (statistic lane/32, query lane%32)
    const int st_id = lane >> 5, st_q = lane & 31;
    const float* st_src = (st_id == 0 ? p.lse : p.delta) + sbase;
    const float st_mul = st_id == 0 ? kLog2e : 1.f;

    auto load_tile = [&](int qt) {
      const int q0 = qt * BQ;
      if (wave < 2) {
        tile_load<T, D>(pre, src + (long)q0 * rs, rs, p.nq - q0, lane);
      } else if (wave == 2) {
        const int qa = q0 + st_q;
        st_pre = qa < p.nq ? st_src[qa] * st_mul : 0.f;
      }
    };
    auto store_tile = [&](int buf) {
      if (wave < 2) {
        tile_store_lds<T, D>(pre, s_row[buf][wave], s_tr[buf][wave], lane);
      } else if (wave == 2) {
        s_stat[buf][st_id][st_q] = st_pre;
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
        f32x16 S = zero16(), dP = zero16();
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          S = mma<T>(frag_row<T, D>(sQ, n, g, ks), kf[ks], S);
          dP = mma<T>(frag_row<T, D>(sdO, n, g, ks), vf[ks], dP);
        }
        const bool need_mask = (q0 + BQ > p.nq) || (CAUSAL && q0 < k0 + 31);
        f32x16 vP, vdS;
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const int m0 = 8 * a + 4 * g;
          const f32x4 l2 = *reinterpret_cast<const f32x4*>(&s_stat[buf][0][m0]);
          const f32x4 dv = *reinterpret_cast<const f32x4*>(&s_stat[buf][1][m0]);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int r = 4 * a + j;
            float pv = exp2_fast(S[r] * c2 - l2[j]);
            if (need_mask) {
              const int qg = q0 + m0 + j;
              const bool ok = qg < p.nq && (!CAUSAL || qg >= kj);
              pv = ok ? pv : 0.f;
            }
            vP[r] = pv;
            vdS[r] = pv * scale * (dP[r] - dv[j]);
          }
        }
        const T* tQ = s_tr[buf][0];
        const T* tdO = s_tr[buf][1];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const V8<T> oP = cvt8<T>(s ? hi8(vP) : lo8(vP));
          const V8<T> oS = cvt8<T>(s ? hi8(vdS) : lo8(vdS));
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            const int col = 32 * dt + n;
            acc_dv[dt] = mma<T>(frag_tr<T, D>(tdO, col, g, s), oP, acc_dv[dt]);
            acc_dk[dt] = mma<T>(frag_tr<T, D>(tQ, col, g, s), oS, acc_dk[dt]);
          }
        }
      }
      if (has_next) store_tile(buf ^ 1);
      __syncthreads();
    }
  }

  if (kvalid) {
    T* dk = p.dk + kbase + (long)kj * rs;
    T* dv = p.dv + kbase + (long)kj * rs;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d = 32 * dt + 8 * a + 4 * g;
        f32x4 x, y;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          x[j] = acc_dk[dt][4 * a + j];
          y[j] = acc_dv[dt][4 * a + j];
        }
        *reinterpret_cast<V4<T>*>(dk + d) = cvt4<T>(x);
        *reinterpret_cast<V4<T>*>(dv + d) = cvt4<T>(y);
      }
    }
  }
}

}  // namespace

template <typename T, int D, bool CAUSAL>
hipError_t launch_bwd(const BwdParams<T>& p, hipStream_t stream) {
  const int nbh = p.batch * p.heads;
  const int nqb = (p.nq + 32 * kWaves - 1) / (32 * kWaves);
  const int nkb = (p.nk + 32 * kWaves - 1) / (32 * kWaves);
  hipLaunchKernelGGL((bwd_q_kernel<T, D, CAUSAL>), dim3(nqb * nbh), dim3(kThreads), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((bwd_k_kernel<T, D, CAUSAL>), dim3(nkb * nbh), dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

#define FHOG_INST(T, D, C) template hipError_t launch_bwd<T, D, C>(const BwdParams<T>&, hipStream_t);
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
