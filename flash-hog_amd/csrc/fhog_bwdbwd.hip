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
// Element-wise form used by passes 3 and 4. With u = dP - D and t = ddS - dD,
//   dP2 - B = dPa + u t - (D dD + B)
// (substitute ddS = t + dD in dP2), so per (query, key) pair
//   dS = scale P u,  dS2 = scale P (dPa + u t - c),  ddP = P t,  c = D dD + B,
// and the common factor `scale` of dS and dS2 is applied once to the dQ2 / dK2
// accumulators instead of per element.
//
// Stage 1 (passes 1-3): a workgroup owns 128 queries (4 waves x 32) of one
// (batch, head) and streams 32-key tiles of K, V, ddK, ddV through an LDS ring
// twice. Score tiles are computed transposed (S^T = K Q^T) so each lane holds
// one query row: row statistics are per-lane scalars and row sums need one
// cross-group add at the end of the sweep. The query-side operands stay in
// registers for the whole sweep.
//
// Stage 2 (pass 4): a workgroup owns 128 keys (4 waves x 32) and streams
// 32-query tiles of Q, dO, ddQ plus their row statistics through an LDS ring.
// Score tiles are S = Q K^T, so each lane holds one key column.
//
// Causal blocks differ in length (query block r sees r + 1 key blocks), so
// both grids issue their blocks longest first: block id -> rank = id / (B H),
// (batch, head) = id % (B H). Workgroups are dispatched round-robin over the
// 8 XCDs (each with its own L2); with B H a multiple of 8, XCD x then receives
// the same eighth of the (batch, head) pairs at every rank, so the blocks that
// stream one (batch, head) share one L2.
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <type_traits>

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

// Depth of the LDS ring: tiles stream NST - 1 iterations ahead of their use.
template <typename T, int D> struct Ring {
  static constexpr int value = (sizeof(T) == 2 && D == 64) ? 4 : 2;
};

// ----------------------------------------------------------------------------
// Stage 1: passes 1-3, tiled over queries.
//
// Sweep 1 (passes 1+2) computes S, ddS, dP and, per row, dD = sum ddS P,
// r2 = sum dP P, r3 = sum dP ddS P, and accumulates P ddV into the ddO
// accumulator; then r1 = sum_j P dPa = <dO_i, (P ddV)_i> and
// B = r1 - dD r2 - D dD + r3. Sweep 2 (pass 3) recomputes S, ddS, dP, dPa and
// adds dS ddK + dS2 K to dQ2 and ddP V to ddO (whose P ddV part came from
// sweep 1). Wave w streams key-side tensor w (K, V, ddK, ddV) global -> LDS,
// without registers, into an NST-deep ring with one barrier per tile.
// ----------------------------------------------------------------------------
template <typename T, int D, bool CAUSAL>
__global__ void __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(Occupancy<T, D>::value, Occupancy<T, D>::value)))
bwdbwd_q_kernel(BwdBwdParams<T> p, int chunk) {
  typedef SwzTile<T, D> G;
  constexpr int KS = D / 16;       // 16-deep steps over the head dim
  constexpr int DT = D / 32;       // 32-wide output column blocks
  constexpr int BQ = 32 * kWaves;  // queries per workgroup
  constexpr int BK = 32;           // keys per streamed tile
  constexpr int NST = Ring<T, D>::value;
  constexpr int kTile = G::kElems * (int)sizeof(T);
  constexpr int kStage = 4 * kTile;  // K, V, ddK, ddV
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

  int kend = p.nk;
  if (CAUSAL) kend = min(kend, qb * BQ + BQ + p.coff);
  // (uniform; saying so keeps the compiler from treating the loops as divergent)
  const int nkt = __builtin_amdgcn_readfirstlane(kend > 0 ? (kend + BK - 1) / BK : 0);  // tiles the workgroup streams
  int wend = p.nk;
  if (CAUSAL) wend = max(0, min(wend, q0 + 32 + p.coff));
  const int wkt = q0 < p.nq ? (wend + BK - 1) / BK : 0;  // tiles with work for this wave

  SwzFrags<T, D> fr;
  fr.init(lane);

  // Wave w streams tensor w; the key sequence is streamed twice (iterations
  // 0 .. nkt-1 and nkt .. 2 nkt - 1).
  const T* src = (wave == 0 ? p.k : wave == 1 ? p.v : wave == 2 ? p.ddk : p.ddv) + kbase;
  const uint32_t row_bytes = (uint32_t)(rsk * (long)sizeof(T));
  TileDma<T, D> dma;
  dma.init(row_bytes, BK, lane);
  const uint32_t lds_kv = lds_base_u32(s_kv);
  const uint32_t lds_wave = lds_kv + wave * kTile;
  const int total = 2 * nkt;
  // Retire the query-side loads here: otherwise the compiler waits for them at
  // their first use inside the loop, and that wait (vmcnt counts every vector
  // load, including the untracked LDS DMAs) would drain the prefetched tiles on
  // every iteration.
  wait_vmem();
  auto issue = [&](int it) {
    const int kt = it < nkt ? it : it - nkt;
    const int nvalid = p.nk - kt * BK;
    const uint32_t dst = lds_wave + (uint32_t)(((uint32_t)it % NST) * kStage);
    const T* gsrc = src + (long)kt * BK * rsk;
    if (nvalid >= BK) {
      dma.issue(dst, gsrc);
    } else {
      TileDma<T, D> part;
      part.init(row_bytes, nvalid, lane);
      part.issue(dst, gsrc);
    }
  };
#pragma unroll
  for (int i = 0; i < NST - 1; ++i)
    if (i < total) issue(i);

  // Waits for tile `it`, then starts streaming tile it + NST - 1 into the stage
  // every wave finished reading in the previous iteration.
  auto advance = [&](int it) {
    wait_tile<NST, G::kLoads>(it, total);
    __syncthreads();
    if (it + NST - 1 < total) issue(it + NST - 1);
  };
  // Masks P on a diagonal or ragged tile (uniform branch).
  auto mask_probs = [&](f32x16& P, int kt) {
    const int k0 = kt * BK;
    const bool need_mask = (k0 + BK > p.nk) || (CAUSAL && k0 + BK - 1 > q0 + p.coff);
    if (need_mask) {
      const int klim = min(p.nk - 1, CAUSAL ? qi + p.coff : p.nk - 1) - k0;  // last visible key, tile-relative
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (crow(r, g) > klim) P[r] = 0.f;
    }
  };

  // ---- sweep 1: dD, r2, r3 and P ddV (into acc_ddo) ----
  f32x16 acc_ddo[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc_ddo[dt] = zero16();
  float dd_acc = 0.f, r2 = 0.f, r3 = 0.f;
  for (int it = 0; it < nkt; ++it) {
    advance(it);
    if (it < wkt) {
      // stage tiles at sa + 0 (K), kTile (V), 2 kTile (ddK), 3 kTile (ddV)
      const uint32_t sa = lds_kv + (uint32_t)(((uint32_t)it % NST) * kStage);
      f32x16 S = zero16(), ddS = zero16(), dP = zero16();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const V8<T> kf = fr.rowf(sa, 0, ks);
        S = mma<T>(kf, qf[ks], S);
        ddS = mma<T>(kf, ddqf[ks], ddS);
        ddS = mma<T>(fr.rowf(sa, 2 * kTile, ks), qf[ks], ddS);
        dP = mma<T>(fr.rowf(sa, kTile, ks), dof[ks], dP);
      }
      f32x16 P;
#pragma unroll
      for (int r = 0; r < 16; ++r) P[r] = exp2_fast(fmaf(S[r], c2, nL2));
      mask_probs(P, it);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float x = ddS[r] * P[r];
        dd_acc += x;
        r3 = fmaf(dP[r], x, r3);
        r2 = fmaf(dP[r], P[r], r2);
      }
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const V8<T> oP = cvt8<T>(s ? hi8(P) : lo8(P));
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc_ddo[dt] = mma<T>(fr.trf(sa, 3 * kTile, dt, s), oP, acc_ddo[dt]);
      }
    }
  }

  // r1 = <dO_i, (P ddV)_i>: the accumulator holds lane = query, registers = columns.
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
  const float nD = -Di, ndD = -dD, nc = -(Di * dD + Bi);

  // ---- sweep 2: dQ2 += P u ddK + P (dPa + u t - c) K (times scale at the end), ddO += P t V ----
  f32x16 acc_dq2[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc_dq2[dt] = zero16();
  for (int it = nkt; it < total; ++it) {
    advance(it);
    const int kt = it - nkt;
    if (kt < wkt) {
      // stage tiles at sa + 0 (K), kTile (V), 2 kTile (ddK), 3 kTile (ddV)
      const uint32_t sa = lds_kv + (uint32_t)(((uint32_t)it % NST) * kStage);
      f32x16 S = zero16(), ddS = zero16(), dP = zero16(), dPa = zero16();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const V8<T> kf = fr.rowf(sa, 0, ks);
        S = mma<T>(kf, qf[ks], S);
        ddS = mma<T>(kf, ddqf[ks], ddS);
        ddS = mma<T>(fr.rowf(sa, 2 * kTile, ks), qf[ks], ddS);
        const V8<T> vf = fr.rowf(sa, kTile, ks);
        dP = mma<T>(vf, dof[ks], dP);
        dPa = mma<T>(fr.rowf(sa, 3 * kTile, ks), dof[ks], dPa);
      }
      f32x16 P;
#pragma unroll
      for (int r = 0; r < 16; ++r) P[r] = exp2_fast(fmaf(S[r], c2, nL2));
      mask_probs(P, kt);
      // one 16-key half at a time: compute, convert, multiply
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        f32x8 vdS, vdS2, vddP;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int r = 8 * s + e;
          const float u = dP[r] + nD;                   // dP - D
          const float t = fmaf(ddS[r], scale, ndD);     // ddS - dD
          const float x = fmaf(u, t, dPa[r]) + nc;      // dP2 - B
          vdS[e] = P[r] * u;
          vdS2[e] = P[r] * x;
          vddP[e] = P[r] * t;
        }
        const V8<T> oS = cvt8<T>(vdS);
        const V8<T> oS2 = cvt8<T>(vdS2);
        const V8<T> odP = cvt8<T>(vddP);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          acc_dq2[dt] = mma<T>(fr.trf(sa, 2 * kTile, dt, s), oS, acc_dq2[dt]);
          acc_dq2[dt] = mma<T>(fr.trf(sa, 0, dt, s), oS2, acc_dq2[dt]);
          acc_ddo[dt] = mma<T>(fr.trf(sa, kTile, dt, s), odP, acc_ddo[dt]);
        }
      }
    }
  }

  if (qvalid) {
    T* dq2 = p.dq2 + qbase + (long)qi * rs;
    T* ddo = p.ddo + qbase + (long)qi * rs;
    // A row that sees exactly one key has a constant softmax: its dQ2 is
    // exactly 0, while the sums above cancel only to rounding of c.
    const bool one_key = (CAUSAL ? min(p.nk, qi + p.coff + 1) : p.nk) == 1;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d = 32 * dt + 8 * a + 4 * g;
        f32x4 x, y;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          x[j] = one_key ? 0.f : acc_dq2[dt][4 * a + j] * scale;
          y[j] = acc_ddo[dt][4 * a + j];
        }
        *reinterpret_cast<V4<T>*>(dq2 + d) = cvt4<T>(x);
        *reinterpret_cast<V4<T>*>(ddo + d) = cvt4<T>(y);
      }
    }
  }
}

// ----------------------------------------------------------------------------
// Stage 2: pass 4, tiled over keys. Waves 0-2 stream the query-side tiles
// (Q, dO, ddQ) global -> LDS; wave 3 streams the tiles' row statistics and
// turns them into the four per-query constants (-L log2(e), -D, -dD,
// -(D dD + B)) in LDS. The loop issues no load the compiler tracks, so its
// only vector-memory waits are the explicit ones.
// ----------------------------------------------------------------------------
template <typename T, int D, bool CAUSAL, bool PRE>
__global__ void __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(Occupancy<T, D>::value, Occupancy<T, D>::value)))
bwdbwd_k_kernel(BwdBwdParams<T> p, int pairs, int chunk) {
  typedef SwzTile<T, D> G;
  constexpr int KS = D / 16;
  constexpr int DT = D / 32;
  constexpr int BKB = 32 * kWaves;  // keys per workgroup
  constexpr int BQ = 32;            // queries per streamed tile
  constexpr int NST = Ring<T, D>::value;
  constexpr int kTile = G::kElems * (int)sizeof(T);
  constexpr int kStat = 4 * BQ * (int)sizeof(float);
  constexpr int kStage = 3 * kTile + kStat;  // Q, dO, ddQ, constants
  __shared__ __attribute__((aligned(1024))) char s_q[NST * kStage];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 31, g = lane >> 5;
  const int nbh = p.batch * p.kv_heads;
  const int nkb = (p.nk + BKB - 1) / BKB;
  // Key block `rank` of pair bh (causal: the longest key columns come first),
  // and with pairs > 0 also a second one (block_pair).
  const GridSlot slot = grid_slot(blockIdx.x, nbh, pairs ? (nkb + 1) / 2 : nkb, chunk);
  const int bh = slot.pair;
  const BlockPair bp = block_pair(slot.rank, nkb, pairs);
  for (int blk = 0; blk < bp.count; ++blk) {
    const int kb = blk == 0 ? bp.first : bp.second;
    if (blk > 0) __syncthreads();  // every wave is done with the previous block's ring
    const int b = bh / p.kv_heads, hk = bh % p.kv_heads;
    const int grp = p.heads / p.kv_heads;  // query heads per key/value head
    const long rs = (long)p.heads * D;      // query-side row stride
    const long rsk = (long)p.kv_heads * D;  // key-side row stride
    // query head hk * grp + gi: tensors at qbase + gi * D, statistics at sbase + gi * nq
    const long qbase = ((long)b * p.nq * p.heads + (long)hk * grp) * D;
    const long kbase = ((long)b * p.nk * p.kv_heads + hk) * D;
    const long sbase = ((long)b * p.heads + (long)hk * grp) * p.nq;
    const int k0 = kb * BKB + wave * 32;
    const int kj = k0 + n;
    const bool kvalid = kj < p.nk;
    const int qfirst = first_contributing_query(p, kj, CAUSAL);

    // Iteration i visits query tile qt_begin + i / grp of query head
    // hk * grp + i % grp (the group reduction of
    // flash_hog/jax/_pallas_gpu_kernel.py:333-370, in one ring).
    const int nqt = (p.nq + BQ - 1) / BQ;
    const int qt_begin = CAUSAL ? max(0, kb * BKB - p.coff) / BQ : 0;

    f32x16 acc_dk2[DT], acc_dv2[DT];
  #pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      acc_dk2[dt] = zero16();
      acc_dv2[dt] = zero16();
    }

    if (qt_begin < nqt) {
      const float scale = p.scale;
      SwzFrags<T, D> fr;
      fr.init(lane);

      const int total = (nqt - qt_begin) * grp;
      const T* src = (wave == 0 ? p.q : wave == 1 ? p.dout : p.ddq) + qbase;
      const uint32_t row_bytes = (uint32_t)(rs * (long)sizeof(T));
      TileDma<T, D> dma;
      dma.init(row_bytes, BQ, lane);
      const uint32_t lds_q = lds_base_u32(s_q);
      const uint32_t lds_wave = lds_q + wave * kTile;
      // Source of the next tile to issue, advanced with the cursor: the next head
      // of the group is D elements on, the next query tile of the first head
      // BQ rows on from the first head.
      const T* gnext = src + (long)qt_begin * BQ * rs;
      const long row_step = (long)BQ * rs - (long)(grp - 1) * D;

      // Wave 3 streams the per-query statistics of each tile with two dword DMAs
      // (lanes 0-31 then 32-63: L and D, then dD and B; rows past nq repeat row
      // nq - 1) into the tile's stage, and once they have landed rewrites them in
      // place as the initial values of the four score accumulators:
      // -L / scale, -dD / scale, -D, -(D dD + B) (-L and -dD when K and ddK carry
      // the scale).
      constexpr int kStatLoads = 4;  // two per lane half
      auto issue_stats = [&](int i, GroupCursor c) {
        // uniform row base plus a per-lane offset; each lane half loads its own tensor
        const uint32_t off = 4u * (uint32_t)min((qt_begin + c.qt) * BQ + n, p.nq - 1);
        const long sb = sbase + (long)c.gi * p.nq;
        const uint32_t dst = lds_base_u32(s_q) + (uint32_t)((i % NST) * kStage + 3 * kTile);
        if (g == 0) {
          dma4s(p.lse + sb, off, dst);
          dma4s(p.ddelta + sb, off, dst + 256);
        } else {
          dma4s(p.delta + sb, off, dst);
          dma4s(p.bstat + sb, off, dst + 256);
        }
      };
      const float inv_scale = 1.0f / scale;
      auto finish_stats = [&](int i) {
        if (g == 0) {
          float* st = reinterpret_cast<float*>(s_q + (i % NST) * kStage + 3 * kTile);
          const float L = st[n], Dq = st[BQ + n], dDq = st[2 * BQ + n], Bq = st[3 * BQ + n];
          st[n] = PRE ? -L : -L * inv_scale;
          st[BQ + n] = PRE ? -dDq : -dDq * inv_scale;
          st[2 * BQ + n] = -Dq;
          st[3 * BQ + n] = -fmaf(Dq, dDq, Bq);
        }
      };
      // Waits (wave 3) until the statistics of tile i have landed: the DMAs of
      // later tiles, at most NST - 2 of them, may still be in flight.
      auto wait_stats = [&](int i) {
        if constexpr (NST >= 3) {
          if (i + NST - 2 < total) {
            wait_vmem_le<(NST - 2) * kStatLoads>();
            return;
          }
        }
        wait_vmem_le<0>();
      };
      auto issue = [&](int i, GroupCursor c) {
        if (wave == 3) {
          issue_stats(i, c);
          return;
        }
        const int q0t = (qt_begin + c.qt) * BQ;
        const uint32_t dst = lds_wave + (uint32_t)((i % NST) * kStage);
        if (q0t + BQ <= p.nq) {
          dma.issue(dst, gnext);
        } else {  // the ragged last query tile (offsets made here: registers are scarce)
          TileDma<T, D> part;
          part.init(row_bytes, p.nq - q0t, lane);
          part.issue(dst, gnext);
        }
      };
      auto advance = [&](GroupCursor& c) {
        gnext += c.gi + 1 == grp ? row_step : (long)D;
        c.next(grp);
      };
      // The ring's first tiles go out before the key-side loads, so that both
      // latencies overlap (this also shortens the loads' live ranges).
      GroupCursor nxt;  // iteration of the next tile to issue
  #pragma unroll
      for (int i = 0; i < NST - 1; ++i)
        if (i < total) {
          issue(i, nxt);
          advance(nxt);
        }

      // Key-side operands (B of the score products).
      V8<T> kf[KS], dkf[KS], vf[KS], dvf[KS];
  #pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const long off = kbase + (long)kj * rsk + 16 * ks + 8 * g;
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
      if constexpr (PRE) {
        // scale is a power of two: K and ddK carry it exactly, so S and ddS come
        // out of the matrix products already scaled (bit-identical to scaling
        // them afterwards) and the element-wise step skips one multiply.
  #pragma unroll
        for (int ks = 0; ks < KS; ++ks)
  #pragma unroll
          for (int e = 0; e < 8; ++e) {
            kf[ks][e] = (T)((float)kf[ks][e] * scale);
            dkf[ks][e] = (T)((float)dkf[ks][e] * scale);
          }
      }
      const float c2 = PRE ? kLog2e : scale * kLog2e;

      // Retire the key-side loads (and with them the first tiles) before the
      // loop: vmcnt counts the untracked LDS DMAs too, so a wait for the loads
      // inside the loop would drain the prefetched tiles.
      wait_vmem();
      if (wave == 3) {
        wait_stats(0);
        finish_stats(0);
      }

      GroupCursor cur;  // iteration i
      for (int i = 0; i < total; ++i, cur.next(grp)) {
        if (wave < 3) wait_tile<NST, G::kLoads>(i, total);
        __syncthreads();
        if (i + NST - 1 < total) {
          issue(i + NST - 1, nxt);
          advance(nxt);
        }
        // Tile i + 1's statistics are read after the next barrier. With a ring
        // of three or more stages their DMA went out two or more iterations
        // ago, and they are finished here, before this tile's work, so that
        // the LDS round trip overlaps wave 3's own products instead of
        // delaying the barrier; with two stages, after this tile's work.
        if constexpr (NST >= 3) {
          if (wave == 3 && i + 1 < total) {
            wait_stats(i + 1);
            finish_stats(i + 1);
          }
        }
        const int q0 = (qt_begin + cur.qt) * BQ;
        const bool active = k0 < p.nk && (!CAUSAL || q0 + BQ - 1 >= k0 - p.coff);
        if (active) {
          const char* st = s_q + (i % NST) * kStage;
          const uint32_t sa = lds_q + (uint32_t)((i % NST) * kStage);  // tiles: Q, dO, ddQ
          const float* sc = reinterpret_cast<const float*>(st + 3 * kTile);
          // The accumulators start at the per-query constants (register r holds
          // query 8 (r / 4) + 4 g + r % 4 of the tile), so they end as
          //   S' = S_raw - L / scale, ddS' = ddS_raw - dD / scale,
          //   u = dP - D, dPa' = dPa - (D dD + B).
          f32x16 S, ddS, dP, dPa;
  #pragma unroll
          for (int a = 0; a < 4; ++a) {
            const int m0 = 8 * a + 4 * g;
            const f32x4 c0 = *reinterpret_cast<const f32x4*>(sc + m0);
            const f32x4 c1 = *reinterpret_cast<const f32x4*>(sc + BQ + m0);
            const f32x4 c2v = *reinterpret_cast<const f32x4*>(sc + 2 * BQ + m0);
            const f32x4 c3 = *reinterpret_cast<const f32x4*>(sc + 3 * BQ + m0);
  #pragma unroll
            for (int j = 0; j < 4; ++j) {
              S[4 * a + j] = c0[j];
              ddS[4 * a + j] = c1[j];
              dP[4 * a + j] = c2v[j];
              dPa[4 * a + j] = c3[j];
            }
          }
  #pragma unroll
          for (int ks = 0; ks < KS; ++ks) {
            const V8<T> qa = fr.rowf(sa, 0, ks);
            const V8<T> dqa = fr.rowf(sa, 2 * kTile, ks);
            const V8<T> doa = fr.rowf(sa, kTile, ks);
            S = mma<T>(qa, kf[ks], S);
            ddS = mma<T>(dqa, kf[ks], ddS);
            ddS = mma<T>(qa, dkf[ks], ddS);
            dP = mma<T>(doa, vf[ks], dP);
            dPa = mma<T>(doa, dvf[ks], dPa);
          }
          f32x16 P;
  #pragma unroll
          for (int r = 0; r < 16; ++r) P[r] = exp2_fast(S[r] * c2);
          const bool need_mask = (q0 + BQ > p.nq) || (CAUSAL && q0 < k0 + 31 - p.coff) || p.nk == 1;
          if (need_mask) {
            // a pair enters iff qfirst <= query < nq
            const int qlo = qfirst - q0, qhi = p.nq - q0;
  #pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int m = crow(r, g);
              if (m < qlo || m >= qhi) P[r] = 0.f;
            }
          }
  #pragma unroll
          for (int s = 0; s < 2; ++s) {
            f32x8 vdS, vdS2, vddP;
  #pragma unroll
            for (int e = 0; e < 8; ++e) {
              const int r = 8 * s + e;
              const float t = PRE ? ddS[r] : ddS[r] * scale;  // ddS - dD
              const float x = fmaf(dP[r], t, dPa[r]);      // dP2 - B
              vdS[e] = P[r] * dP[r];
              vdS2[e] = P[r] * x;
              vddP[e] = P[r] * t;
            }
            const V8<T> oS = cvt8<T>(vdS);
            const V8<T> oS2 = cvt8<T>(vdS2);
            const V8<T> odP = cvt8<T>(vddP);
  #pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
              acc_dk2[dt] = mma<T>(fr.trf(sa, 2 * kTile, dt, s), oS, acc_dk2[dt]);
              acc_dk2[dt] = mma<T>(fr.trf(sa, 0, dt, s), oS2, acc_dk2[dt]);
              acc_dv2[dt] = mma<T>(fr.trf(sa, kTile, dt, s), odP, acc_dv2[dt]);
            }
          }
        }
        if constexpr (NST < 3) {
          if (wave == 3 && i + 1 < total) {
            wait_stats(i + 1);
            finish_stats(i + 1);
          }
        }
      }
    }

    if (kvalid) {
      const float scale = p.scale;
      T* dk2 = p.dk2 + kbase + (long)kj * rsk;
      T* dv2 = p.dv2 + kbase + (long)kj * rsk;
  #pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
  #pragma unroll
        for (int a = 0; a < 4; ++a) {
          const int d = 32 * dt + 8 * a + 4 * g;
          f32x4 x, y;
  #pragma unroll
          for (int j = 0; j < 4; ++j) {
            x[j] = acc_dk2[dt][4 * a + j] * scale;
            y[j] = acc_dv2[dt][4 * a + j];
          }
          *reinterpret_cast<V4<T>*>(dk2 + d) = cvt4<T>(x);
          *reinterpret_cast<V4<T>*>(dv2 + d) = cvt4<T>(y);
        }
      }
    }
  }
}

}  // namespace

// Stage 1 for 2-byte types at D = 64 runs the kernel with 32 queries per
// wave at one wave per SIMD, a hand-scheduled sweep and a persistent grid
// (fhog_bwdbwd_q32.hip) unless FLASH_HOG_STAGE1=fused selects the fused
// kernel (16 queries per wave, two waves per SIMD), which serves D = 128 and
// 256. Both give the same results to rounding; the q32 kernel is 3-6 % faster
// on every D = 64 configuration measured (179 against 185 us at B4 N2048 H16
// causal bf16, 137 against 146 us at B8 N1000 H12 fp16). Read at every launch,
// so a process can switch between them.
inline bool stage1_fused_selected() {
  const char* v = std::getenv("FLASH_HOG_STAGE1");
  return v != nullptr && std::strcmp(v, "fused") == 0;
}

// Stage 2 for bf16 at D = 64 runs bwdbwd_k_kernel below (32 keys per wave,
// two waves per SIMD) unless FLASH_HOG_STAGE2=k32 selects the kernel with a
// generated sweep at one wave per SIMD (fhog_bwdbwd_k32.hip). Both give the
// same results to rounding; at B4 N2048 H16 D64 causal bf16 the compiled
// kernel is about 10 % faster. Read at every launch.
inline bool stage2_k32_selected() {
  const char* v = std::getenv("FLASH_HOG_STAGE2");
  return v != nullptr && std::strcmp(v, "k32") == 0;
}

template <typename T, int D, bool CAUSAL>
hipError_t launch_bwdbwd(const BwdBwdParams<T>& p, hipStream_t stream, int stages) {
  const int nqb = (p.nq + 32 * kWaves - 1) / (32 * kWaves);
  const int nkb = (p.nk + 32 * kWaves - 1) / (32 * kWaves);
  if (stages & 1) {
    hipError_t e;
    if constexpr (sizeof(T) == 2 && D == 64) {
      e = stage1_fused_selected() ? launch_bwdbwd_stage1_fused<T, D, CAUSAL>(p, stream)
                                  : launch_bwdbwd_stage1_q32<T, CAUSAL>(p, stream);
    } else if constexpr (sizeof(T) == 2) {
      e = launch_bwdbwd_stage1_fused<T, D, CAUSAL>(p, stream);
    } else {
      const int npairs = p.batch * p.heads;
      hipLaunchKernelGGL((bwdbwd_q_kernel<T, D, CAUSAL>), dim3(nqb * npairs), dim3(kThreads), 0, stream, p,
                         grid_chunk(npairs, nqb, resident_workgroups(Occupancy<T, D>::value)));
      e = hipGetLastError();
    }
    if (e != hipSuccess) return e;
  }
  if (stages & 2) {
    if constexpr (sizeof(T) == 2 && D >= 128) {
      return launch_bwdbwd_stage2_k16<T, D, CAUSAL>(p, stream);
    } else {
      if constexpr (std::is_same_v<T, __bf16> && D == 64) {
        if (stage2_k32_selected()) return launch_bwdbwd_stage2_k32<CAUSAL>(p, stream);
      }
      // Pair causal key blocks when the grid outnumbers the resident workgroups.
      const int npairs = p.batch * p.kv_heads;
      const int resident = resident_workgroups(Occupancy<T, D>::value);
      const int pairs = block_pairing(CAUSAL, nkb, npairs, resident, Occupancy<T, D>::value);
      const int nranks = pairs ? (nkb + 1) / 2 : nkb;
      const int chunk = grid_chunk(npairs, nranks, resident);
      const dim3 grid(nranks * npairs);
      int e2;
      if (std::is_same_v<T, __bf16> && std::frexp(p.scale, &e2) == 0.5f)  // scale = 2^(e2 - 1)
        hipLaunchKernelGGL((bwdbwd_k_kernel<T, D, CAUSAL, std::is_same_v<T, __bf16>>), grid, dim3(kThreads), 0, stream,
                           p, pairs, chunk);
      else
        hipLaunchKernelGGL((bwdbwd_k_kernel<T, D, CAUSAL, false>), grid, dim3(kThreads), 0, stream, p, pairs, chunk);
      return hipGetLastError();
    }
  }
  return hipSuccess;
}

#define FHOG_INST(T, D, C) template hipError_t launch_bwdbwd<T, D, C>(const BwdBwdParams<T>&, hipStream_t, int);
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
