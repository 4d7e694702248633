// First-order attention backward on gfx950, atomic free:
//   D  = rowsum(O * dO),  P = exp(scale Q K^T - L),  dP = dO V^T,
//   dS = scale P (dP - D),  dQ = dS K,  dK = dS^T Q,  dV = P^T dO.
// Replaces the cuDNN backward that the reference calls through
// flash_hog/jax/_attention_impl.py:242-261; the equations are those of
// flash_hog/_jax_refs/jax_impl.py:142-191 (attn_bwd).
//
// Kernel 1 (tiled over queries) computes D for its rows, writes it, and
// accumulates dQ while streaming K and V. Kernel 2 (tiled over keys) reads L
// and D and accumulates dK and dV while streaming Q and dO. Both stream their
// tiles global -> LDS (no registers) through a 4-stage ring of XOR-swizzled
// tiles with one barrier per tile, issue causal blocks longest first with
// (batch, head) as the minor index, mask only diagonal and ragged tiles, and
// apply the factor `scale` of dS once to the dQ / dK accumulators. Score tiles
// use the orientations of the double backward (fhog_bwdbwd.hip): transposed
// in kernel 1 (row statistics are per-lane scalars), direct in kernel 2,
// whose score accumulators start at the per-query constants -L / scale and -D
// so that the MFMAs fold them in.
#include <cstdlib>
#include <cstring>

#include "fhog_device.h"
#include "fhog_params.h"

namespace fhog {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kStages = 4;  // 3 stages: 2.6 % slower at B4 N2048 H16

// Waves per SIMD the register allocator is asked to allow: two for 2-byte
// types at D = 64 and 128 (at D = 128 the dQ kernel takes 238 VGPRs and the
// dK/dV kernel, in two column passes, 242; first backward at B4 N2048 H16
// causal 495 -> 403-417 us), one otherwise.
template <typename T, int D> struct Occupancy {
  static constexpr int value = (sizeof(T) == 2 && D <= 128) ? 2 : 1;
};
// Whether the dK/dV kernel runs as two passes over halves of the output
// columns (each forming the full scores): at D = 256 all columns'
// accumulators beside the resident K and V spilled 740 bytes per lane; for
// 2-byte types at D = 128 they took 401 registers (one wave per SIMD) against
// 242 per pass (two waves).
template <typename T, int D> struct KSplit {
  static constexpr bool value = D > 128 || (sizeof(T) == 2 && D == 128);
};


template <typename T, int D, bool CAUSAL>
__global__ void __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(Occupancy<T, D>::value, Occupancy<T, D>::value)))
bwd_q_kernel(BwdParams<T> p, int chunk) {
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

  V8<T> qf[KS], dof[KS];
  float dpart = 0.f;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const long off = qbase + (long)qi * rs + 16 * ks + 8 * g;
    if (qvalid) {
      qf[ks] = *reinterpret_cast<const V8<T>*>(p.q + off);
      dof[ks] = *reinterpret_cast<const V8<T>*>(p.dout + off);
      const V8<T> of = *reinterpret_cast<const V8<T>*>(p.o + off);
      if constexpr (sizeof(T) == 2) {
        dpart = dot8<T>(of, dof[ks], dpart);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) dpart += (float)of[e] * (float)dof[ks][e];
      }
    } else {
      qf[ks] = zero8<T>();
      dof[ks] = zero8<T>();
    }
  }
  const float Di = xgroup_sum(dpart);
  const float nL2 = qvalid ? -p.lse[sbase + qi] * kLog2e : 0.f;

  int kend = p.nk;
  if (CAUSAL) kend = min(kend, qb * BQ + BQ + p.coff);
  // (uniform; saying so keeps the compiler from treating the loop as divergent)
  const int nkt = __builtin_amdgcn_readfirstlane(kend > 0 ? (kend + BK - 1) / BK : 0);
  int wend = p.nk;
  if (CAUSAL) wend = max(0, min(wend, q0 + 32 + p.coff));
  const int wkt = q0 < p.nq ? (wend + BK - 1) / BK : 0;

  const float scale = p.scale;
  const float c2 = scale * kLog2e;
  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = zero16();
  // At D = 64 the dP accumulator starts at -D (a loop-invariant register
  // tuple read by each tile's first dP product), so it ends as u = dP - D and
  // the element-wise step saves 16 subtractions per tile (first backward at
  // B4 N2048 H16 150.5 -> 146.6 us). At larger D the tuple's 16 registers
  // would spill, and u is formed per element.
  constexpr bool kU0 = D == 64;
  f32x16 u0 = zero16();
  if constexpr (kU0) {
#pragma unroll
    for (int r = 0; r < 16; ++r) u0[r] = -Di;
  }

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

  // Retire the query-side loads before the ring starts (see fwd_kernel).
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
      f32x16 S = zero16(), u = u0;  // u: dP - D at D = 64, dP otherwise
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        S = mma<T>(fr.rowf(sa, 0, ks), qf[ks], S);
        u = mma<T>(fr.rowf(sa, kTile, ks), dof[ks], u);
      }
      f32x16 P;
#pragma unroll
      for (int r = 0; r < 16; ++r) P[r] = exp2_fast(fmaf(S[r], c2, nL2));
      const int k0 = kt * BK;
      if ((k0 + BK > p.nk) || (CAUSAL && k0 + BK - 1 > q0 + p.coff)) {
        const int klim = min(p.nk - 1, CAUSAL ? qi + p.coff : p.nk - 1) - k0;  // last visible key, tile-relative
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (crow(r, g) > klim) P[r] = 0.f;
      }
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        f32x8 vdS;
#pragma unroll
        for (int e = 0; e < 8; ++e) vdS[e] = P[8 * s + e] * (kU0 ? u[8 * s + e] : u[8 * s + e] - Di);  // dS / scale
        const V8<T> oS = cvt8<T>(vdS);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[dt] = mma<T>(fr.trf(sa, 0, dt, s), oS, acc[dt]);
      }
    }
  }

  if (qvalid) {
    T* dq = p.dq + qbase + (long)qi * rs;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        f32x4 x;
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = acc[dt][4 * a + j] * scale;
        *reinterpret_cast<V4<T>*>(dq + 32 * dt + 8 * a + 4 * g) = cvt4<T>(x);
      }
    }
    if (g == 0) p.delta[sbase + qi] = Di;
  }
}

// Kernel 2: tiled over keys. Waves 0-1 load the two halves of each Q tile,
// waves 2-3 those of each dO tile; wave 3 also loads the tile's L and D with
// dword DMAs and, once they have landed, rewrites them in LDS as the initial
// values of the S and dP accumulators (-L / scale and -D).
//
// With KSplit (2-byte types at D = 128 and 256) the launcher runs the kernel
// twice, for output column blocks [C0, C0 + DTO) with C0 = 0 and D / 64, each
// pass forming the full scores again, so that the dK and dV accumulators of
// half the columns fit beside the resident K and V.
template <typename T, int D, bool CAUSAL, int C0>
__global__ void __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(Occupancy<T, D>::value, Occupancy<T, D>::value)))
bwd_k_kernel(BwdParams<T> p, int chunk) {
  typedef SwzTile<T, D> G;
  constexpr int KS = D / 16;
  constexpr int DTO = KSplit<T, D>::value ? D / 64 : D / 32;  // 32-column output blocks of this pass
  constexpr int BKB = 32 * kWaves;
  constexpr int BQ = 32;
  constexpr int NST = kStages;
  constexpr int kTile = G::kElems * (int)sizeof(T);
  // Statistics area: two 256-byte rows (L, D of the tile's 32 queries, then a
  // copy the upper half-wave writes and nothing reads).
  constexpr int kStatRow = 64 * (int)sizeof(float);
  constexpr int kSR = kStatRow / (int)sizeof(float);
  constexpr int kStage = 2 * kTile + 2 * kStatRow;  // Q, dO, statistics
  constexpr int kPer = G::kLoads / 2;
  constexpr int kStatWave = 3;
  __shared__ __attribute__((aligned(1024))) char s_q[NST * kStage];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 31, g = lane >> 5;
  const int nbh = p.batch * p.kv_heads;
  const int nkb = (p.nk + 32 * kWaves - 1) / (32 * kWaves);
  const GridSlot gs = grid_slot(blockIdx.x, nbh, nkb, chunk);
  const int kb = gs.rank;  // causal: the longest key columns come first
  const int bh = gs.pair;
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
  const float scale = p.scale;

  // Iteration i visits query tile qt_begin + i / grp of query head
  // hk * grp + i % grp: the heads of a group share each tile's causal bounds.
  const int nqt = (p.nq + BQ - 1) / BQ;
  const int qt_begin = CAUSAL ? max(0, kb * BKB - p.coff) / BQ : 0;
  const int total = nqt > qt_begin ? (nqt - qt_begin) * grp : 0;

  f32x16 acc_dk[DTO], acc_dv[DTO];
#pragma unroll
  for (int dt = 0; dt < DTO; ++dt) acc_dk[dt] = acc_dv[dt] = zero16();

  if (total > 0) {
    V8<T> kf[KS], vf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const long off = kbase + (long)kj * rsk + 16 * ks + 8 * g;
      kf[ks] = kvalid ? *reinterpret_cast<const V8<T>*>(p.k + off) : zero8<T>();
      vf[ks] = kvalid ? *reinterpret_cast<const V8<T>*>(p.v + off) : zero8<T>();
    }
    const float c2 = scale * kLog2e;
    const float inv_scale = 1.0f / scale;

    SwzFrags<T, D> fr;
    fr.init(lane);
    const int tensor = wave >> 1;  // 0 = Q, 1 = dO
    const T* src = (tensor == 0 ? p.q : p.dout) + qbase;
    const uint32_t row_bytes = (uint32_t)(rs * (long)sizeof(T));
    TileDma<T, D, kPer> dma;
    dma.init(row_bytes, BQ, lane, kPer * (wave & 1));
    const uint32_t lds0 = lds_base_u32(s_q);
    // Sources of the next tile to issue, advanced with the cursor: the next
    // head of the group is D elements (statistics: nq) on, the next query tile
    // of the first head BQ rows on from the first head.
    const T* gnext = src + (long)qt_begin * BQ * rs;
    const long row_step = (long)BQ * rs - (long)(grp - 1) * D;
    const long soff0 = sbase + (long)qt_begin * BQ;
    const float* lnext = p.lse + soff0;
    const float* dnext = p.delta + soff0;
    const long stat_step = (long)BQ - (long)(grp - 1) * p.nq;
    auto issue = [&](int i, GroupCursor c) {
      const int q0t = (qt_begin + c.qt) * BQ;
      const uint32_t stage = lds0 + (uint32_t)(((uint32_t)i % NST) * kStage);
      const int nvalid = p.nq - q0t;
      if (nvalid >= BQ) {
        dma.issue(stage + tensor * kTile, gnext);
      } else {
        TileDma<T, D, kPer> part;
        part.init(row_bytes, nvalid, lane, kPer * (wave & 1));
        part.issue(stage + tensor * kTile, gnext);
      }
      if (wave == kStatWave) {
        // lane l reads query q0t + (l % 32); rows past nq repeat row nq - 1
        const uint32_t voff = 4u * (uint32_t)min(n, nvalid - 1);
        dma4s(lnext, voff, stage + 2 * kTile);
        dma4s(dnext, voff, stage + 2 * kTile + kStatRow);
      }
    };
    auto advance = [&](GroupCursor& c) {
      const bool last = c.gi + 1 == grp;
      gnext += last ? row_step : (long)D;
      lnext += last ? stat_step : (long)p.nq;
      dnext += last ? stat_step : (long)p.nq;
      c.next(grp);
    };
    auto finish_stats = [&](int i) {
      if (wave == kStatWave && g == 0) {
        float* st = reinterpret_cast<float*>(s_q + ((uint32_t)i % NST) * kStage + 2 * kTile);
        st[n] = -st[n] * inv_scale;
        st[kSR + n] = -st[kSR + n];
      }
    };
    // Waits for tile i (the statistics wave issues two more loads per tile).
    auto wait_for = [&](int i) {
      if (wave == kStatWave)
        wait_tile<NST, kPer + 2>(i, total);
      else
        wait_tile<NST, kPer>(i, total);
    };

    // Retire the key-side loads before the ring starts (see fwd_kernel).
    wait_vmem();
    GroupCursor nxt;  // iteration of the next tile to issue
#pragma unroll
    for (int i = 0; i < NST - 1; ++i)
      if (i < total) {
        issue(i, nxt);
        advance(nxt);
      }

    GroupCursor cur;  // iteration i
    for (int i = 0; i < total; ++i, cur.next(grp)) {
      wait_for(i);
      finish_stats(i);
      __syncthreads();
      if (i + NST - 1 < total) {
        issue(i + NST - 1, nxt);
        advance(nxt);
      }
      const int q0 = (qt_begin + cur.qt) * BQ;
      const bool active = k0 < p.nk && (!CAUSAL || q0 + BQ - 1 >= k0 - p.coff);
      if (active) {
        const char* st = s_q + ((uint32_t)i % NST) * kStage;
        const uint32_t sa = lds0 + (uint32_t)(((uint32_t)i % NST) * kStage);  // Q at 0, dO at kTile
        const float* sc = reinterpret_cast<const float*>(st + 2 * kTile);
        // S' = S_raw - L / scale, u = dP - D (register r holds query
        // 8 (r / 4) + 4 g + r % 4 of the tile)
        f32x16 S, dP;
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const int m0 = 8 * a + 4 * g;
          const f32x4 v0 = *reinterpret_cast<const f32x4*>(sc + m0);
          const f32x4 v1 = *reinterpret_cast<const f32x4*>(sc + kSR + m0);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            S[4 * a + j] = v0[j];
            dP[4 * a + j] = v1[j];
          }
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          S = mma<T>(fr.rowf(sa, 0, ks), kf[ks], S);
          dP = mma<T>(fr.rowf(sa, kTile, ks), vf[ks], dP);
        }
        f32x16 P;
#pragma unroll
        for (int r = 0; r < 16; ++r) P[r] = exp2_fast(S[r] * c2);
        if ((q0 + BQ > p.nq) || (CAUSAL && q0 < k0 + 31 - p.coff)) {
          // visible iff query >= key - coff (causal) and query < nq
          const int qlo = (CAUSAL ? kj - p.coff : 0) - q0, qhi = p.nq - q0;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int m = crow(r, g);
            if (m < qlo || m >= qhi) P[r] = 0.f;
          }
        }
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          f32x8 vdS;
#pragma unroll
          for (int e = 0; e < 8; ++e) vdS[e] = P[8 * s + e] * dP[8 * s + e];  // dS / scale
          const V8<T> oP = cvt8<T>(s ? hi8(P) : lo8(P));
          const V8<T> oS = cvt8<T>(vdS);
#pragma unroll
          for (int dt = 0; dt < DTO; ++dt) {
            acc_dv[dt] = mma<T>(fr.trf(sa, kTile, C0 + dt, s), oP, acc_dv[dt]);
            acc_dk[dt] = mma<T>(fr.trf(sa, 0, C0 + dt, s), oS, acc_dk[dt]);
          }
        }
      }
    }
  }

  if (kvalid) {
    T* dk = p.dk + kbase + (long)kj * rsk;
    T* dv = p.dv + kbase + (long)kj * rsk;
#pragma unroll
    for (int dt = 0; dt < DTO; ++dt) {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d = 32 * (C0 + dt) + 8 * a + 4 * g;
        f32x4 x, y;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          x[j] = acc_dk[dt][4 * a + j] * scale;
          y[j] = acc_dv[dt][4 * a + j];
        }
        *reinterpret_cast<V4<T>*>(dk + d) = cvt4<T>(x);
        *reinterpret_cast<V4<T>*>(dv + d) = cvt4<T>(y);
      }
    }
  }
}

}  // namespace

// The first backward for 2-byte types at D = 64 has two kernels for each
// half of its work: dK/dV in bwd_k_kernel above or in bwd_k64_kernel
// (fhog_bwd_k64.hip: 64 keys per wave at one wave per SIMD, generated sweep),
// dQ in bwd_q_kernel above or in bwd_q64_kernel (fhog_bwd_q64.hip, the same
// with 64 queries per wave). A one-wave kernel runs one 256-row block per CU
// at a time and gains nothing when a CU is left alone, so it is taken when
// its grid fills whole rounds of the resident workgroups (or at least six),
// and the compiled kernel, whose second workgroup per CU runs faster alone,
// otherwise: first backward at B4 N2048 H16 causal bf16 138.7-140.7 us with
// both one-wave kernels against 148.5-149.1 with both compiled ones, while
// at B8 N2048 H12 causal (1.5 rounds) the one-wave dQ kernel took 258
// against 241 us. FLASH_HOG_BWD (dK/dV) and FLASH_HOG_BWDQ (dQ) = compiled or
// k64 / q64 force a kernel; read at every launch.
inline bool one_wave_grid(int workgroups, int resident) {
  return resident > 0 && workgroups > 0 && (workgroups % resident == 0 || workgroups >= 6 * resident);
}
inline bool one_wave_selected(const char* var, const char* name, int nb, int npairs, bool causal) {
  const char* v = std::getenv(var);
  if (v != nullptr && std::strcmp(v, name) == 0) return true;
  if (v != nullptr && std::strcmp(v, "compiled") == 0) return false;
  const int resident = resident_workgroups(1);
  const int pairs = block_pairing(causal, nb, npairs, resident, 1);
  return one_wave_grid((pairs ? (nb + 1) / 2 : nb) * npairs, resident);
}

template <typename T, int D, bool CAUSAL>
hipError_t launch_bwd(const BwdParams<T>& p, hipStream_t stream) {
  const int nqb = (p.nq + 32 * kWaves - 1) / (32 * kWaves);
  const int nkb = (p.nk + 32 * kWaves - 1) / (32 * kWaves);
  const int resident = resident_workgroups(Occupancy<T, D>::value);
  const int nq_pairs = p.batch * p.heads, nk_pairs = p.batch * p.kv_heads;
  hipError_t e = hipSuccess;
  if constexpr (sizeof(T) == 2 && D == 64) {
    if (one_wave_selected("FLASH_HOG_BWDQ", "q64", (p.nq + 255) / 256, nq_pairs, CAUSAL))
      e = launch_bwd_q64<T, CAUSAL>(p, stream);
    else
      hipLaunchKernelGGL((bwd_q_kernel<T, D, CAUSAL>), dim3(nqb * nq_pairs), dim3(kThreads), 0, stream, p,
                         grid_chunk(nq_pairs, nqb, resident));
  } else {
    hipLaunchKernelGGL((bwd_q_kernel<T, D, CAUSAL>), dim3(nqb * nq_pairs), dim3(kThreads), 0, stream, p,
                       grid_chunk(nq_pairs, nqb, resident));
  }
  if (e == hipSuccess) e = hipGetLastError();
  if (e != hipSuccess) return e;
  if constexpr (sizeof(T) == 2 && D == 64) {
    if (one_wave_selected("FLASH_HOG_BWD", "k64", (p.nk + 255) / 256, nk_pairs, CAUSAL))
      return launch_bwd_k64<T, CAUSAL>(p, stream);
  }
  hipLaunchKernelGGL((bwd_k_kernel<T, D, CAUSAL, 0>), dim3(nkb * nk_pairs), dim3(kThreads), 0, stream, p,
                     grid_chunk(nk_pairs, nkb, resident));
  if constexpr (KSplit<T, D>::value) {
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL((bwd_k_kernel<T, D, CAUSAL, D / 64>), dim3(nkb * nk_pairs), dim3(kThreads), 0, stream, p,
                       grid_chunk(nk_pairs, nkb, resident));
  }
  return hipGetLastError();
}

#define FHOG_INST(T, D, C) template hipError_t launch_bwd<T, D, C>(const BwdParams<T>&, hipStream_t);
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
