// Stage 2 of the Flash-HOG double backward (pass 4: dK2, dV2) with 16 keys per
// wave, for 2-byte types at D = 128 and 256. The math is that of fhog_bwdbwd.hip's
// stage 2 (flash_hog/_jax_refs/jax_impl.py:273-336, the pass split of
// flash_hog/jax/_pallas_gpu_kernel.py:309-391): per (query, key) pair, with
// the per-query constants folded into the accumulator start values,
//   dS = scale P u,  dS2 = scale P (dPa + u t - c),  ddP = P t,
//   dK2 = sum_i dS ddQ + dS2 Q,  dV2 = sum_i ddP dO.
//
// Why 16 keys per wave at D = 128. With 32 keys per wave the two 32 x 128
// accumulators (128 registers) and the four resident key-side operands (128)
// already exceed the 256 registers of a wave that shares its SIMD, so that
// kernel runs one wave per SIMD and nothing overlaps one wave's matrix work
// with another's vector work. With 16 keys the same state takes half the
// registers, two waves share each SIMD, and each query-side tile is read from
// LDS by twice as many waves (the price: twice the LDS bytes per product).
// At D = 64 the 32-key kernel already runs two waves per SIMD and is faster.
// At D = 256 the state of 16 keys takes 446 registers: one wave per SIMD, one
// workgroup per CU (the 32-key kernel spilled 1400 bytes per lane there).
//
// 16x16x32 layouts (fhog_device.h): score tiles are S = Q K^T (queries x
// keys, two 16-query halves per 32-query tile); lane (n, g) holds key n and
// queries 4 g + i of each half, so a pair of halves fed back as the B operand
// of an output product contracts over queries in the permuted order
// k' = 8 g + e -> query 4 g + e (e < 4) or 16 + 4 g + e - 4 (e >= 4), and the
// query-side tile is read transposed in the same order (SwzFrags16::trf).
// Output accumulators hold columns 16 db + 4 g + i of key n.
#include <cmath>
#include <type_traits>

#include "fhog_device.h"
#include "fhog_params.h"

namespace fhog {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kKeys = 16;  // keys per wave

// The four score tiles of a 32-query tile for one wave (two 16-query halves
// each), started at the per-query constants: S' = S - L / scale,
// ddS' = ddS - dD / scale (-L and -dD when K and ddK carry the scale),
// u = dP - D, dPa' = dPa - (D dD + B).
struct Scores16 {
  f32x4 S[2], ddS[2], dP[2], dPa[2];
};

template <typename T, int D, bool CAUSAL, bool PRE>
__global__ void __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(D <= 128 ? 2 : 1, D <= 128 ? 2 : 1)))
bwdbwd_k16_kernel(BwdBwdParams<T> p, int chunk) {
  typedef SwzTile<T, D> G;
  constexpr int KS = D / 32;             // 32-deep steps over the head dim (score products)
  constexpr int DB = D / 16;             // 16-wide output column blocks
  constexpr int BKB = kKeys * kWaves;    // keys per workgroup
  constexpr int BQ = 32;                 // queries per streamed tile
  // Each iteration's scores are formed and then finished (the registers of a
  // second score set, for a software-pipelined loop, are not there at
  // D = 128). Three stages of 24.5 KiB fit two workgroups per CU at D = 128,
  // three of 48.5 KiB one at D = 256.
  constexpr int NST = 3;
  constexpr int kTile = G::kElems * (int)sizeof(T);
  constexpr int kStat = 4 * BQ * (int)sizeof(float);
  constexpr int kStage = 3 * kTile + kStat;  // Q, dO, ddQ, constants
  constexpr int kStatLoads = 2;
  __shared__ __attribute__((aligned(1024))) char s_q[NST * kStage];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int nbh = p.batch * p.kv_heads;
  const int nkb = (p.nk + BKB - 1) / BKB;
  // Key block `rank` of pair bh, the longest (causal) first. Unlike the 32-key
  // kernel, this one does not pair key block r with its mirror: its grids have
  // twice as many blocks, and rank-major order balances them better (stage 2
  // at B2 N8192 H16 D128: 2.54-2.57 ms unpaired against 2.64 ms paired).
  const GridSlot slot = grid_slot(blockIdx.x, nbh, nkb, chunk);
  const int bh = slot.pair;
  {
    const int kb = slot.rank;
    const int b = bh / p.kv_heads, hk = bh % p.kv_heads;
    const int grp = p.heads / p.kv_heads;  // query heads per key/value head
    const long rs = (long)p.heads * D;      // query-side row stride
    const long rsk = (long)p.kv_heads * D;  // key-side row stride
    const long qbase = ((long)b * p.nq * p.heads + (long)hk * grp) * D;
    const long kbase = ((long)b * p.nk * p.kv_heads + hk) * D;
    const long sbase = ((long)b * p.heads + (long)hk * grp) * p.nq;
    const int k0 = kb * BKB + wave * kKeys;
    const int kj = k0 + n;
    const bool kvalid = kj < p.nk;
    const int qfirst = first_contributing_query(p, kj, CAUSAL);

    // Iteration i visits query tile qt_begin + i / grp of query head
    // hk * grp + i % grp (the group reduction of _pallas_gpu_kernel.py:333-370).
    const int nqt = (p.nq + BQ - 1) / BQ;
    const int qt_begin = CAUSAL ? max(0, kb * BKB - p.coff) / BQ : 0;
    const int total = __builtin_amdgcn_readfirstlane(qt_begin < nqt ? (nqt - qt_begin) * grp : 0);

    f32x4 acc_dk2[DB], acc_dv2[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) acc_dk2[db] = acc_dv2[db] = zero4();

    if (total > 0) {
      const float scale = p.scale;
      const float c2 = PRE ? kLog2e : scale * kLog2e;
      const float inv_scale = 1.0f / scale;
      SwzFrags16<T, D> fr;
      fr.init(lane);
      const bool loader = wave < 3;
      const T* src = (wave == 0 ? p.q : wave == 1 ? p.dout : p.ddq) + qbase;
      const uint32_t row_bytes = (uint32_t)(rs * (long)sizeof(T));
      TileDma<T, D, G::kLoads, kSwzRows> dma;
      dma.init(row_bytes, BQ, lane);
      const uint32_t lds_q = lds_base_u32(s_q);
      const uint32_t lds_wave = lds_q + wave * kTile;
      auto slot_addr = [&](int i) { return lds_q + (uint32_t)(((uint32_t)i % NST) * kStage); };
      auto stats = [&](int i) {
        return reinterpret_cast<float*>(s_q + ((uint32_t)i % NST) * kStage + 3 * kTile);
      };

      // Loader waves stream tensor `wave` of iteration i; wave 3 streams the
      // iteration's row statistics (lanes 0-31 then 32-63: L and D, then dD
      // and B; rows past nq repeat row nq - 1).
      auto issue = [&](int i, GroupCursor c) {
        const int q0t = (qt_begin + c.qt) * BQ;
        if (loader) {
          const int nvalid = p.nq - q0t;
          const uint32_t dst = lds_wave + (uint32_t)(((uint32_t)i % NST) * kStage);
          const T* gsrc = src + (long)c.gi * D + (long)q0t * rs;
          if (nvalid >= BQ) {
            dma.issue(dst, gsrc);
          } else {
            TileDma<T, D, G::kLoads, kSwzRows> part;
            part.init(row_bytes, nvalid, lane);
            part.issue(dst, gsrc);
          }
        } else {
          const uint32_t off = 4u * (uint32_t)min(q0t + (lane & 31), p.nq - 1);
          const long sb = sbase + (long)c.gi * p.nq;
          const uint32_t dst = lds_q + (uint32_t)(((uint32_t)i % NST) * kStage + 3 * kTile);
          // each lane half loads its own tensors (the base must be uniform)
          if (lane < 32) {
            dma4s(p.lse + sb, off, dst);
            dma4s(p.ddelta + sb, off, dst + 256);
          } else {
            dma4s(p.delta + sb, off, dst);
            dma4s(p.bstat + sb, off, dst + 256);
          }
        }
      };
      int hi = -1;  // last iteration issued
      GroupCursor nxt_issue;
      auto issue_next = [&]() {
        issue(++hi, nxt_issue);
        nxt_issue.next(grp);
      };
      // The ring's first tiles go out before the key-side loads, so that both
      // latencies overlap.
#pragma unroll
      for (int k = 0; k < NST - 1; ++k)
        if (k < total) issue_next();

      // Key-side operands (B of the score products): key n, columns 32 ks + 8 g .. +7.
      V8<T> kf[KS], dkf[KS], vf[KS], dvf[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const long off = kbase + (long)kj * rsk + 32 * ks + 8 * g;
        if (kvalid) {
          kf[ks] = *reinterpret_cast<const V8<T>*>(p.k + off);
          dkf[ks] = *reinterpret_cast<const V8<T>*>(p.ddk + off);
          vf[ks] = *reinterpret_cast<const V8<T>*>(p.v + off);
          dvf[ks] = *reinterpret_cast<const V8<T>*>(p.ddv + off);
        } else {
          kf[ks] = dkf[ks] = vf[ks] = dvf[ks] = zero8<T>();
        }
      }
      if constexpr (PRE) {
        // scale is a power of two: K and ddK carry it exactly (see stage 2 in
        // fhog_bwdbwd.hip).
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            kf[ks][e] = (T)((float)kf[ks][e] * scale);
            dkf[ks][e] = (T)((float)dkf[ks][e] * scale);
          }
      }
      // Retire the key-side loads (and the ring's first tiles) before the loop:
      // vmcnt also counts the untracked LDS DMAs.
      wait_vmem();

      // Waits until this wave's loads of iteration i have landed (the loads
      // of later iterations, at most NST - 2 of them, may stay in flight).
      auto wait_own = [&](int i) {
        const int ahead = hi - i;
        if (loader) {
          if (ahead >= 1)
            wait_vmem_le<G::kLoads>();
          else
            wait_vmem_le<0>();
        } else {
          if (ahead >= 1)
            wait_vmem_le<kStatLoads>();
          else
            wait_vmem_le<0>();
        }
      };
      static_assert(NST == 3, "wait_own assumes at most one iteration issued past the one awaited");
      // Wave 3 rewrites the landed statistics of iteration i as the
      // accumulator start values; they are read after a later barrier.
      auto convert_stats = [&](int i) {
        if (loader || i >= total) return;
        wait_own(i);
        if (lane < 32) {
          float* st = stats(i);
          const float L = st[lane], Dq = st[BQ + lane], dDq = st[2 * BQ + lane], Bq = st[3 * BQ + lane];
          st[lane] = PRE ? -L : -L * inv_scale;
          st[BQ + lane] = PRE ? -dDq : -dDq * inv_scale;
          st[2 * BQ + lane] = -Dq;
          st[3 * BQ + lane] = -fmaf(Dq, dDq, Bq);
        }
      };
      // Makes iteration i's tiles visible to every wave and starts the load
      // of iteration i + 2 into the stage of iteration i - 1, which every
      // wave finished reading before this barrier.
      auto advance = [&](int i) {
        if (loader) wait_own(i);
        __syncthreads();
        if (hi + 1 < total) issue_next();
      };

      struct Iter {
        int q0;
        bool active;
      };
      auto iter_info = [&](GroupCursor c) {
        Iter it;
        it.q0 = (qt_begin + c.qt) * BQ;
        it.active = k0 < p.nk && (!CAUSAL || it.q0 + BQ - 1 >= k0 - p.coff);
        return it;
      };

      // Score tiles of iteration i (Q at 0, dO at kTile, ddQ at 2 kTile,
      // constants at 3 kTile of its stage).
      auto scores = [&](int i, Scores16& sc) {
        const uint32_t sa = slot_addr(i);
        const float* st = stats(i);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int m0 = 16 * h + 4 * g;
          sc.S[h] = *reinterpret_cast<const f32x4*>(st + m0);
          sc.ddS[h] = *reinterpret_cast<const f32x4*>(st + BQ + m0);
          sc.dP[h] = *reinterpret_cast<const f32x4*>(st + 2 * BQ + m0);
          sc.dPa[h] = *reinterpret_cast<const f32x4*>(st + 3 * BQ + m0);
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) {
            const V8<T> qa = fr.rowf(sa, 0, h, ks);
            const V8<T> dqa = fr.rowf(sa, 2 * kTile, h, ks);
            sc.S[h] = mma16<T>(qa, kf[ks], sc.S[h]);
            sc.ddS[h] = mma16<T>(dqa, kf[ks], sc.ddS[h]);
            sc.ddS[h] = mma16<T>(qa, dkf[ks], sc.ddS[h]);
            const V8<T> doa = fr.rowf(sa, kTile, h, ks);
            sc.dP[h] = mma16<T>(doa, vf[ks], sc.dP[h]);
            sc.dPa[h] = mma16<T>(doa, dvf[ks], sc.dPa[h]);
          }
        }
      };
      // Element-wise step and output products of iteration i. Element e of
      // the permuted query order is half e / 4, register e % 4 (tile-relative
      // query 16 (e / 4) + 4 g + e % 4); with MASK, queries outside
      // [qlo, qhi) get P = 0.
      auto finish = [&](int i, const Scores16& sc, const Iter& it, auto mask_tag) {
        constexpr bool MASK = decltype(mask_tag)::value;
        const uint32_t sa = slot_addr(i);
        const int qlo = qfirst - it.q0, qhi = p.nq - it.q0;
        f32x8 vS, vS2, vP;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int h = e >> 2, r = e & 3;
          float P = exp2_fast(sc.S[h][r] * c2);
          if (MASK) {
            const int m = 16 * h + 4 * g + r;
            if (m < qlo || m >= qhi) P = 0.f;
          }
          const float t = PRE ? sc.ddS[h][r] : sc.ddS[h][r] * scale;  // ddS - dD
          const float x = fmaf(sc.dP[h][r], t, sc.dPa[h][r]);         // dP2 - B
          vS[e] = P * sc.dP[h][r];
          vS2[e] = P * x;
          vP[e] = P * t;
        }
        const V8<T> oS = cvt8<T>(vS), oS2 = cvt8<T>(vS2), odP = cvt8<T>(vP);
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          acc_dk2[db] = mma16<T>(fr.trf(sa, 2 * kTile, db), oS, acc_dk2[db]);
          acc_dk2[db] = mma16<T>(fr.trf(sa, 0, db), oS2, acc_dk2[db]);
          acc_dv2[db] = mma16<T>(fr.trf(sa, kTile, db), odP, acc_dv2[db]);
        }
      };

      GroupCursor cur;  // iteration i
      convert_stats(0);
      // One iteration: scores and finish of i (masked where a query lies
      // past nq or before the causal diagonal).
      auto plain_step = [&](int i, auto mask_tag) {
        advance(i);
        convert_stats(i + 1);
        const Iter it = iter_info(cur);
        if (it.active) {
          Scores16 sc;
          scores(i, sc);
          finish(i, sc, it, mask_tag);
        }
        cur.next(grp);
      };
      for (int i = 0; i < total; ++i) plain_step(i, std::true_type{});
    }

    if (kvalid) {
      const float scale = p.scale;
      T* dk2 = p.dk2 + kbase + (long)kj * rsk;
      T* dv2 = p.dv2 + kbase + (long)kj * rsk;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const int d = 16 * db + 4 * g;  // this lane's four output columns
        f32x4 x;
#pragma unroll
        for (int r = 0; r < 4; ++r) x[r] = acc_dk2[db][r] * scale;
        *reinterpret_cast<V4<T>*>(dk2 + d) = cvt4<T>(x);
        *reinterpret_cast<V4<T>*>(dv2 + d) = cvt4<T>(acc_dv2[db]);
      }
    }
  }
}

}  // namespace

template <typename T, int D, bool CAUSAL>
hipError_t launch_bwdbwd_stage2_k16(const BwdBwdParams<T>& p, hipStream_t stream) {
  static_assert(sizeof(T) == 2, "2-byte types only");
  const int nkb = (p.nk + kKeys * kWaves - 1) / (kKeys * kWaves);
  const int npairs = p.batch * p.kv_heads;
  const int chunk = grid_chunk(npairs, nkb, resident_workgroups(D <= 128 ? 2 : 1));
  const dim3 grid(nkb * npairs);
  int e2;
  if (std::is_same_v<T, __bf16> && std::frexp(p.scale, &e2) == 0.5f)  // scale = 2^(e2 - 1)
    hipLaunchKernelGGL((bwdbwd_k16_kernel<T, D, CAUSAL, std::is_same_v<T, __bf16>>), grid, dim3(kThreads), 0,
                       stream, p, chunk);
  else
    hipLaunchKernelGGL((bwdbwd_k16_kernel<T, D, CAUSAL, false>), grid, dim3(kThreads), 0, stream, p, chunk);
  return hipGetLastError();
}

#define FHOG_INST(T, D, C) template hipError_t launch_bwdbwd_stage2_k16<T, D, C>(const BwdBwdParams<T>&, hipStream_t);
FHOG_INST(__bf16, 128, true)
FHOG_INST(__bf16, 128, false)
FHOG_INST(_Float16, 128, true)
FHOG_INST(_Float16, 128, false)
FHOG_INST(__bf16, 256, true)
FHOG_INST(__bf16, 256, false)
FHOG_INST(_Float16, 256, true)
FHOG_INST(_Float16, 256, false)
#undef FHOG_INST

}  // namespace fhog
