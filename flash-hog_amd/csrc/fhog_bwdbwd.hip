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

// Waves per SIMD the register allocator is asked to allow: two for 2-byte
// types at D = 64 (so one wave's matrix work overlaps the other's vector work),
// one otherwise.
template <typename T, int D> struct Occupancy {
  static constexpr int value = (sizeof(T) == 2 && D == 64) ? 2 : 1;
};

// ----------------------------------------------------------------------------
// Stage 1: passes 1-3, tiled over queries.
//
// Sweep 1 (passes 1+2) computes S, ddS, dP and, per row, dD = sum ddS P,
// r2 = sum dP P, r3 = sum dP ddS P, and accumulates u = P ddV into the ddO
// accumulator; then r1 = sum_j P dPa = <dO_i, u_i> and
// B = r1 - dD r2 - D dD + r3. Sweep 2 (pass 3) recomputes S, ddS, dP, dPa and
// adds dS ddK + dS2 K to dQ2 and ddP V to ddO (whose P ddV part came from
// sweep 1). Key-side tiles go global -> LDS directly (no registers) into a
// two-stage ring with one barrier per tile.
// ----------------------------------------------------------------------------
template <typename T, int D, bool CAUSAL>
__global__ void __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(Occupancy<T, D>::value, Occupancy<T, D>::value)))
bwdbwd_q_kernel(BwdBwdParams<T> p) {
  typedef SwzTile<T, D> G;
  constexpr int KS = D / 16;       // 16-deep steps over the head dim
  constexpr int DT = D / 32;       // 32-wide output column blocks
  constexpr int BQ = 32 * kWaves;  // queries per workgroup
  constexpr int BK = 32;           // keys per streamed tile
  // [stage][tensor]: 0 = K, 1 = V, 2 = ddK, 3 = ddV
  __shared__ __attribute__((aligned(1024))) T s_kv[2][4][G::kElems];

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
  const float scale = p.scale;
  const float c2 = scale * kLog2e;
  const float Di = xgroup_sum(dpart);
  const float nL2 = qvalid ? -p.lse[sbase + qi] * kLog2e : 0.f;
  const float nsD = -scale * Di;

  int kend = p.nk;
  if (CAUSAL) kend = min(kend, qb * BQ + BQ);
  const int nkt = (kend + BK - 1) / BK;                   // tiles the workgroup streams
  int wend = p.nk;
  if (CAUSAL) wend = min(wend, q0 + 32);
  const int wkt = q0 < p.nq ? (wend + BK - 1) / BK : 0;  // tiles with work for this wave

  const T* src = (wave == 0 ? p.k : wave == 1 ? p.v : wave == 2 ? p.ddk : p.ddv) + kbase;
  const int total = 2 * nkt;
  tile_load_lds<T, D>(s_kv[0][wave], src, rs, p.nk, lane);

  // Waits for tile `it`, then starts streaming tile it + 1 (the key sequence is
  // streamed twice) into the other stage.
  auto advance = [&](int it) {
    wait_vmem();
    __syncthreads();
    if (it + 1 < total) {
      const int kn = it + 1 < nkt ? it + 1 : it + 1 - nkt;
      tile_load_lds<T, D>(s_kv[(it + 1) & 1][wave], src + (long)kn * BK * rs, rs, p.nk - kn * BK, lane);
    }
  };
  // P of the tile at stage `buf` (key tile kt), masked on diagonal / ragged tiles.
  auto probs = [&](const f32x16& S, int kt) {
    const int k0 = kt * BK;
    const bool need_mask = (k0 + BK > p.nk) || (CAUSAL && k0 + BK - 1 > q0);
    const int klim = min(p.nk - 1, CAUSAL ? qi : p.nk - 1) - k0;  // last visible key, tile-relative
    f32x16 P;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float pv = exp2_fast(fmaf(S[r], c2, nL2));
      P[r] = (need_mask && crow(r, g) > klim) ? 0.f : pv;
    }
    return P;
  };

  // ---- sweep 1: dD, r2, r3 and u = P ddV (into acc_ddo) ----
  f32x16 acc_ddo[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc_ddo[dt] = zero16();
  float dd_acc = 0.f, r2 = 0.f, r3 = 0.f;
  for (int it = 0; it < nkt; ++it) {
    advance(it);
    if (it < wkt) {
      const T* sK = s_kv[it & 1][0];
      const T* sV = s_kv[it & 1][1];
      const T* sdK = s_kv[it & 1][2];
      const T* sdV = s_kv[it & 1][3];
      f32x16 S = zero16(), ddS = zero16(), dP = zero16();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const V8<T> kf = frag_row_swz<T, D>(sK, n, g, ks);
        S = mma<T>(kf, qf[ks], S);
        ddS = mma<T>(kf, ddqf[ks], ddS);
        ddS = mma<T>(frag_row_swz<T, D>(sdK, n, g, ks), qf[ks], ddS);
        dP = mma<T>(frag_row_swz<T, D>(sV, n, g, ks), dof[ks], dP);
      }
      const f32x16 P = probs(S, it);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        dd_acc = fmaf(ddS[r], P[r], dd_acc);
        r2 = fmaf(dP[r], P[r], r2);
        r3 = fmaf(dP[r] * ddS[r], P[r], r3);
      }
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const V8<T> oP = cvt8<T>(s ? hi8(P) : lo8(P));
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
          acc_ddo[dt] = mma<T>(frag_tr_swz<T, D>(sdV, 32 * dt, lane, s), oP, acc_ddo[dt]);
      }
    }
  }

  // r1 = <dO_i, u_i>: u is in the accumulator layout (lane = query, registers = columns).
  float r1 = 0.f;
  if (qvalid) {
    const T* dorow = p.dout + qbase + (long)qi * rs;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const V4<T> x = *reinterpret_cast<const V4<T>*>(dorow + 32 * dt + 8 * a + 4 * g);
#pragma unroll
        for (int j = 0; j < 4; ++j) r1 = fmaf((float)x[j], acc_ddo[dt][4 * a + j], r1);
      }
    }
  }
  const float dD = xgroup_sum(dd_acc) * scale;
  const float Bi = xgroup_sum(r1) - dD * xgroup_sum(r2) - Di * dD + xgroup_sum(r3) * scale;
  if (qvalid && g == 0) {
    p.delta[sbase + qi] = Di;
    p.ddelta[sbase + qi] = dD;
    p.bstat[sbase + qi] = Bi;
  }
  const float ndd = -dD, nsB = -scale * Bi;

  // ---- sweep 2: dQ2 += dS ddK + dS2 K, ddO += ddP V ----
  f32x16 acc_dq2[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc_dq2[dt] = zero16();
  for (int it = nkt; it < total; ++it) {
    advance(it);
    const int kt = it - nkt;
    if (kt < wkt) {
      const T* sK = s_kv[it & 1][0];
      const T* sV = s_kv[it & 1][1];
      const T* sdK = s_kv[it & 1][2];
      const T* sdV = s_kv[it & 1][3];
      f32x16 S = zero16(), ddS = zero16(), dP = zero16(), dPa = zero16();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const V8<T> kf = frag_row_swz<T, D>(sK, n, g, ks);
        S = mma<T>(kf, qf[ks], S);
        ddS = mma<T>(kf, ddqf[ks], ddS);
        ddS = mma<T>(frag_row_swz<T, D>(sdK, n, g, ks), qf[ks], ddS);
        dP = mma<T>(frag_row_swz<T, D>(sV, n, g, ks), dof[ks], dP);
        dPa = mma<T>(frag_row_swz<T, D>(sdV, n, g, ks), dof[ks], dPa);
      }
      const f32x16 P = probs(S, kt);
      // one 16-key half at a time: compute, convert, multiply
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        f32x8 vdS, vdS2, vddP;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int r = 8 * s + e;
          const float t = fmaf(ddS[r], scale, ndd);            // ddS - dD
          float w = fmaf(dP[r], t, dPa[r]);                     // dPa + dP (ddS - dD)
          w = fmaf(ddS[r], nsD, w);                             //   - ddS D  = dP2
          vdS[e] = P[r] * fmaf(dP[r], scale, nsD);              // scale P (dP - D)
          vdS2[e] = P[r] * fmaf(w, scale, nsB);                 // scale P (dP2 - B)
          vddP[e] = P[r] * t;                                   // P (ddS - dD)
        }
        const V8<T> oS = cvt8<T>(vdS);
        const V8<T> oS2 = cvt8<T>(vdS2);
        const V8<T> odP = cvt8<T>(vddP);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          acc_dq2[dt] = mma<T>(frag_tr_swz<T, D>(sdK, 32 * dt, lane, s), oS, acc_dq2[dt]);
          acc_dq2[dt] = mma<T>(frag_tr_swz<T, D>(sK, 32 * dt, lane, s), oS2, acc_dq2[dt]);
          acc_ddo[dt] = mma<T>(frag_tr_swz<T, D>(sV, 32 * dt, lane, s), odP, acc_ddo[dt]);
        }
      }
    }
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
  }
}

// ----------------------------------------------------------------------------
// Stage 2: pass 4, tiled over keys. Query-side tiles (Q, dO, ddQ) go
// global -> LDS directly; the four row statistics of each query tile are
// staged through registers as -L log2(e), -scale D, -dD, -scale B.
// ----------------------------------------------------------------------------
template <typename T, int D, bool CAUSAL>
__global__ void __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(Occupancy<T, D>::value, Occupancy<T, D>::value)))
bwdbwd_k_kernel(BwdBwdParams<T> p) {
  typedef SwzTile<T, D> G;
  constexpr int KS = D / 16;
  constexpr int DT = D / 32;
  constexpr int BKB = 32 * kWaves;  // keys per workgroup
  constexpr int BQ = 32;            // queries per streamed tile
  // [stage][tensor]: 0 = Q, 1 = dO, 2 = ddQ
  __shared__ __attribute__((aligned(1024))) T s_q[2][3][G::kElems];
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

    // Wave w streams query-side tensor w (w < 3); every wave stages statistic w.
    const T* src = (wave == 0 ? p.q : wave == 1 ? p.dout : p.ddq) + qbase;
    const float* st_src = (wave == 0 ? p.lse : wave == 1 ? p.delta : wave == 2 ? p.ddelta : p.bstat) + sbase;
    const float st_mul = wave == 0 ? -kLog2e : wave == 1 ? -scale : wave == 2 ? -1.f : -scale;
    auto load_stat = [&](int qt) {
      const int q = qt * BQ + n;
      return (g == 0 && q < p.nq) ? st_src[q] * st_mul : 0.f;
    };

    if (wave < 3) tile_load_lds<T, D>(s_q[0][wave], src + (long)qt_begin * BQ * rs, rs, p.nq - qt_begin * BQ, lane);
    {
      const float v = load_stat(qt_begin);
      if (g == 0) s_stat[0][wave][n] = v;
    }

    for (int qt = qt_begin; qt < nqt; ++qt) {
      const int buf = (qt - qt_begin) & 1;
      const bool has_next = qt + 1 < nqt;
      wait_vmem();
      __syncthreads();
      float st_next = 0.f;
      if (has_next) {
        st_next = load_stat(qt + 1);
        if (wave < 3)
          tile_load_lds<T, D>(s_q[buf ^ 1][wave], src + (long)(qt + 1) * BQ * rs, rs, p.nq - (qt + 1) * BQ, lane);
      }
      const int q0 = qt * BQ;
      const bool active = k0 < p.nk && (!CAUSAL || q0 + BQ - 1 >= k0);
      if (active) {
        const T* sQ = s_q[buf][0];
        const T* sdO = s_q[buf][1];
        const T* sdQ = s_q[buf][2];
        f32x16 S = zero16(), ddS = zero16(), dP = zero16(), dPa = zero16();
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const V8<T> qa = frag_row_swz<T, D>(sQ, n, g, ks);
          const V8<T> dqa = frag_row_swz<T, D>(sdQ, n, g, ks);
          const V8<T> doa = frag_row_swz<T, D>(sdO, n, g, ks);
          S = mma<T>(qa, kf[ks], S);
          ddS = mma<T>(dqa, kf[ks], ddS);
          ddS = mma<T>(qa, dkf[ks], ddS);
          dP = mma<T>(doa, vf[ks], dP);
          dPa = mma<T>(doa, dvf[ks], dPa);
        }
        const bool need_mask = (q0 + BQ > p.nq) || (CAUSAL && q0 < k0 + 31);
        // visible iff query >= qmin (causal) and query < nq
        const int qlo = (CAUSAL ? kj : 0) - q0, qhi = p.nq - q0;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          f32x8 vdS, vdS2, vddP;
#pragma unroll
          for (int ah = 0; ah < 2; ++ah) {
            const int a = 2 * s + ah;
            const int m0 = 8 * a + 4 * g;
            const f32x4 nl2 = *reinterpret_cast<const f32x4*>(&s_stat[buf][0][m0]);
            const f32x4 nsd = *reinterpret_cast<const f32x4*>(&s_stat[buf][1][m0]);
            const f32x4 ndd = *reinterpret_cast<const f32x4*>(&s_stat[buf][2][m0]);
            const f32x4 nsb = *reinterpret_cast<const f32x4*>(&s_stat[buf][3][m0]);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int r = 4 * a + j, e = 4 * ah + j;
              float pv = exp2_fast(fmaf(S[r], c2, nl2[j]));
              if (need_mask) pv = (m0 + j < qlo || m0 + j >= qhi) ? 0.f : pv;
              const float t = fmaf(ddS[r], scale, ndd[j]);
              float w = fmaf(dP[r], t, dPa[r]);
              w = fmaf(ddS[r], nsd[j], w);
              vdS[e] = pv * fmaf(dP[r], scale, nsd[j]);
              vdS2[e] = pv * fmaf(w, scale, nsb[j]);
              vddP[e] = pv * t;
            }
          }
          const V8<T> oS = cvt8<T>(vdS);
          const V8<T> oS2 = cvt8<T>(vdS2);
          const V8<T> odP = cvt8<T>(vddP);
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            acc_dk2[dt] = mma<T>(frag_tr_swz<T, D>(sdQ, 32 * dt, lane, s), oS, acc_dk2[dt]);
            acc_dk2[dt] = mma<T>(frag_tr_swz<T, D>(sQ, 32 * dt, lane, s), oS2, acc_dk2[dt]);
            acc_dv2[dt] = mma<T>(frag_tr_swz<T, D>(sdO, 32 * dt, lane, s), odP, acc_dv2[dt]);
          }
        }
      }
      if (has_next && g == 0) s_stat[buf ^ 1][wave][n] = st_next;
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
