// Stage 1 of the Flash-HOG double backward (passes 1-3) in one sweep over the
// keys, for 2-byte types at D = 128 and 256, and at D = 64 when
// FLASH_HOG_STAGE1=fused selects it over fhog_bwdbwd_q32.hip (fhog_bwdbwd.hip
// holds the two-sweep stage 1 used for fp32, and stage 2). The math follows
// flash_hog/_jax_refs/jax_impl.py:273-336 and the pass split of
// flash_hog/jax/_pallas_gpu_kernel.py:149-278; outputs and row statistics are
// those of fhog_bwdbwd.hip's stage 1.
//
// One sweep. dD and B are only known at the end of the sweep, but they enter
// dQ2 and ddO as per-row factors of sums that can be accumulated separately.
// With u = dP - D, x = P ddS (ddS including its scale) and
// X = P (dPa + ddS u):
//   dQ2 = scale (sum_j P u ddK + sum_j X K - dD sum_j P u K - c sum_j P K),
//   ddO = sum_j P ddV + sum_j x V - dD O,                c = D dD + B,
// because P (dP2 - B) = X - dD P u - c P, ddP = x - dD P and sum_j P V = O.
// The row statistic comes from two more per-pair sums: summing
// P (dP2 - B) = X - dD P u - c P over the keys (sum_j P = 1, and B is
// sum_j P dP2, flash_hog/jax/_pallas_gpu_kernel.py:209-210) gives
//   c = sum_j X - dD sum_j P u,   B = c - D dD,
// both sums taken over the fp32 values before any rounding. (c also equals
// <dO, ddO>, but ddO accumulates P and x rounded to T, and the subtraction
// D dD cancels most of c, so that form left B off by up to 1e-2 of |c|: at
// D = 256 with four queries that put dK2 at 2.2e-2 of its largest entry.)
// Every key tile is streamed once; per
// tile a wave forms the five score products (S, ddS twice, dP, dPa), one exp
// per pair, and six output products into four accumulators (dQ2 part,
// sum P u K, sum P K, ddO part). The dP accumulator starts at -D, so it ends
// as u.
//
// Rounding. The ddO accumulator takes x rounded to T (bf16 or fp16) as the
// operand of sum_j x V, and sum_j x V - dD O cancels to the small
// sum_j x (V_j - O) when a row's keys carry similar P ddS. So the epilogue
// subtracts dD' O with dD' = sum_j T(x_j), the dD of the rounded values (four
// v_dot2 with ones per 32-key tile), and the cancellation leaves no rounding
// residue of x; dD itself, B and dQ2 keep the unrounded sum. Against a CPU
// model of this kernel's roundings over 40 random bf16 problems, this halves
// the worst relative error of ddO, dQ2 and dK2 (0.020 -> 0.009 where rows see
// few keys, as with N_K = 34 under a causal mask).
//
// Rows that see exactly one key (the first row of a causal problem, or every
// row when N_K = 1). There P = 1, dS = dS2 = ddP = 0, so dQ2 = 0 and ddO =
// ddV_0 exactly. With one key x = dD' and O = V_0, so ddO comes out exact;
// dQ2's sums cancel only up to the rounding of X and x (about 1e-2 at
// unit-size inputs where the exact value is 0), and the epilogue writes
// dQ2 = 0 for such rows.
//
// Sixteen queries per wave. The five accumulators of 32 queries would not fit
// beside the score tiles in the 256 registers of a wave that shares its SIMD
// with another, and two co-resident waves are what overlaps one wave's matrix
// work with the other's vector work. So a wave owns 16 queries and uses the
// 16x16x32 matrix instruction (v_mfma_f32_16x16x32_{bf16,f16}). At D = 128 this
// still fits two waves per SIMD when each tile's scores are formed and then
// finished (no pipelining): 2.78 ms at B2 N8192 H16 against 3.90 ms for the
// two-sweep stage 1 at one wave per SIMD. Layouts:
//   A (16 x 32): lane holds A[m = l % 16][k = 8 (l / 16) + e],   e = 0..7
//   B (32 x 16): lane holds B[k = 8 (l / 16) + e][n = l % 16]
//   C (16 x 16): lane holds C[m = 4 (l / 16) + i][n = l % 16],   i = 0..3
// Score tiles are transposed (keys x queries, two 16-key C tiles per 32-key
// tile), so each lane holds one query; a C tile pair fed back as the B
// operand of an output product contracts over keys in the permuted order
// k' = 8 g + e -> key 4 g + e (e < 4) or 16 + 4 g + e - 4 (e >= 4), and the
// A operand (the key-side tile, transposed) is read with two
// ds_read_b64_tr_b16 in the same order.
#include <cmath>
#include <type_traits>

#include "fhog_device.h"
#include "fhog_params.h"

namespace fhog {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kQ = 16;  // queries per wave

// The four score tiles of a 32-key tile for one wave (two 16-key C tiles
// each), transposed (keys x queries): S, ddS (without its scale unless Q and
// ddQ carry it), dP, dPa.
struct Scores {
  f32x4 S[2], ddS[2], dP[2], dPa[2];
};

template <typename T, int D, bool CAUSAL, bool PRE>
__global__ void __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(D <= 128 ? 2 : 1, D <= 128 ? 2 : 1)))
bwdbwd_q_fused_kernel(BwdBwdParams<T> p, int chunk) {
  typedef SwzTile<T, D> G;
  constexpr int KS = D / 32;       // 32-deep steps over the head dim (score products)
  constexpr int DB = D / 16;       // 16-wide output column blocks
  constexpr int BQ = kQ * kWaves;  // queries per workgroup
  constexpr int BK = 32;           // keys per streamed tile
  // D = 64: a software-pipelined loop (the scores of tile t + 1 beside the
  // element-wise step of tile t) over a 4-stage ring (64 KiB); D = 128: the
  // accumulators and operands take twice the registers, so each tile's
  // scores are formed and finished in turn, over a 2-stage ring (64 KiB).
  // D = 256: the same at one wave per SIMD (512 registers), over a 2-stage
  // ring of 128 KiB (one workgroup per CU).
  constexpr bool PIPE = D == 64;
  constexpr int NST = PIPE ? 4 : 2;  // tiles t (finishing), t + 1 (scores), two in flight
  constexpr int kTile = G::kElems * (int)sizeof(T);
  constexpr int kStage = 4 * kTile;  // K, V, ddK, ddV
  __shared__ __attribute__((aligned(1024))) char s_kv[NST * kStage];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;
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
  const int q0 = qb * BQ + wave * kQ;
  const int qi = q0 + n;
  const bool qvalid = qi < p.nq;

  // Keys [0, kend) are visible to some query of the workgroup, [0, wend) to
  // some query of this wave.
  int kend = p.nk;
  if (CAUSAL) kend = min(kend, qb * BQ + BQ + p.coff);
  // (uniform; saying so keeps the compiler from treating the loop as divergent)
  const int nkt = __builtin_amdgcn_readfirstlane(kend > 0 ? (kend + BK - 1) / BK : 0);
  int wend = p.nk;
  if (CAUSAL) wend = max(0, min(wend, q0 + kQ + p.coff));
  const int wkt = q0 < p.nq ? (wend + BK - 1) / BK : 0;  // tiles with work for this wave

  SwzFrags16<T, D> fr;
  fr.init(lane);

  // Wave w streams key-side tensor w (K, V, ddK, ddV) into an NST-stage ring.
  const T* src = (wave == 0 ? p.k : wave == 1 ? p.v : wave == 2 ? p.ddk : p.ddv) + kbase;
  const T* gnext = src;  // source of the next tile to issue (tiles are issued in order)
  const uint32_t row_bytes = (uint32_t)(rsk * (long)sizeof(T));
  TileDma<T, D, G::kLoads, kSwzRows> dma;
  dma.init(row_bytes, BK, lane);
  const uint32_t lds_kv = lds_base_u32(s_kv);
  const uint32_t lds_wave = lds_kv + wave * kTile;
  auto issue = [&](int kt) {
    const int nvalid = p.nk - kt * BK;
    const uint32_t dst = lds_wave + (uint32_t)(((uint32_t)kt % NST) * kStage);
    const T* gsrc = gnext;
    gnext += BK * rsk;
    if (nvalid >= BK) {
      dma.issue(dst, gsrc);
    } else {
      TileDma<T, D, G::kLoads, kSwzRows> part;
      part.init(row_bytes, nvalid, lane);
      part.issue(dst, gsrc);
    }
  };
  // The ring's first NST - 1 tiles: all but the last go out before the
  // query-side loads and the last once the query side has been used. The
  // compiler does not count the LDS DMAs (they are inline assembly), so its
  // waits for the query side also wait for every DMA issued before them; the
  // loop's own waits count DMAs and are only made stricter by older loads.
  int hi = -1;  // last tile issued
#pragma unroll
  for (int i = 0; i < NST - 2; ++i)
    if (i < nkt) issue(++hi);

  // Query-side operands (B of the score products), D_i = <O_i, dO_i> and the
  // logsumexp, in one batch of loads. A lane past the last query loads the
  // last query's row: its own results are never stored, and a matrix product
  // column or row sum of one query never mixes in another's, so finite
  // values are all it needs.
  const long roff = qbase + (long)min(qi, p.nq - 1) * rs;
  V8<T> qf[KS], ddqf[KS], dof[KS], of[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const long off = roff + 32 * ks + 8 * g;
    qf[ks] = *reinterpret_cast<const V8<T>*>(p.q + off);
    ddqf[ks] = *reinterpret_cast<const V8<T>*>(p.ddq + off);
    dof[ks] = *reinterpret_cast<const V8<T>*>(p.dout + off);
    of[ks] = *reinterpret_cast<const V8<T>*>(p.o + off);
  }
  const float lse = p.lse[sbase + min(qi, p.nq - 1)];
  float dpart = 0.f;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
#pragma unroll
    for (int e = 0; e < 8; ++e) dpart += (float)of[ks][e] * (float)dof[ks][e];
  const float scale = p.scale;
  if constexpr (PRE) {
    // scale is a power of two: Q and ddQ carry it exactly, so S and ddS come
    // out of the matrix products already scaled (bit-identical to scaling them
    // afterwards) and the element-wise step skips one multiply.
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        qf[ks][e] = (T)((float)qf[ks][e] * scale);
        ddqf[ks][e] = (T)((float)ddqf[ks][e] * scale);
      }
  }
  const float c2 = PRE ? kLog2e : scale * kLog2e;
  const float Di = group4_sum(dpart);
  const float nD = -Di;
  const float nL2 = -lse * kLog2e;
  // Everything the loop takes from the query side is final before the last
  // prologue tile is issued (the empty statements pin the order, and the
  // memory clobber keeps the loads above them).
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) asm volatile("" ::"v"(qf[ks]), "v"(ddqf[ks]), "v"(dof[ks]));
  asm volatile("" ::"v"(nD), "v"(nL2) : "memory");
  if (NST - 2 < nkt) issue(++hi);

  f32x4 acc_a[DB], acc_s[DB], acc_p[DB], acc_o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc_a[db] = acc_s[db] = acc_p[db] = acc_o[db] = zero4();
  float dd_acc = 0.f;  // dD = sum P ddS over this lane's keys
  float ddr_acc = 0.f;  // the same sum over P ddS rounded to T, as the ddO products take it
  float xs_acc = 0.f;   // sum X over this lane's keys
  float pu_acc = 0.f;   // sum P u over this lane's keys
  const f32x4 init_u = {nD, nD, nD, nD};

  // Score tiles of the key tile in slot sa (K at 0, V at kTile, ddK at
  // 2 kTile, ddV at 3 kTile); kb = 16-key half. sc.dP ends as u = dP - D.
  auto scores = [&](uint32_t sa, Scores& sc) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      sc.S[kb] = sc.ddS[kb] = sc.dPa[kb] = zero4();
      sc.dP[kb] = init_u;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const V8<T> kf = fr.rowf(sa, 0, kb, ks);
        sc.S[kb] = mma16<T>(kf, qf[ks], sc.S[kb]);
        sc.ddS[kb] = mma16<T>(kf, ddqf[ks], sc.ddS[kb]);
        sc.ddS[kb] = mma16<T>(fr.rowf(sa, 2 * kTile, kb, ks), qf[ks], sc.ddS[kb]);
        sc.dP[kb] = mma16<T>(fr.rowf(sa, kTile, kb, ks), dof[ks], sc.dP[kb]);
        sc.dPa[kb] = mma16<T>(fr.rowf(sa, 3 * kTile, kb, ks), dof[ks], sc.dPa[kb]);
      }
    }
  };
  // Element-wise step and output products of the key tile in slot sa whose
  // scores are sc. Element e of the permuted key order is C tile e / 4,
  // register e % 4 (tile-relative key 16 (e / 4) + 4 g + e % 4); keys past
  // klim are masked when MASK.
  auto finish = [&](uint32_t sa, const Scores& sc, int klim, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    f32x8 vP, vx, vu, vX;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int kb = e >> 2, i = e & 3;
      float P = exp2_fast(fmaf(sc.S[kb][i], c2, nL2));
      if (MASK && 16 * kb + 4 * g + i > klim) P = 0.f;
      const float x = PRE ? P * sc.ddS[kb][i] : P * (sc.ddS[kb][i] * scale);  // P ddS
      const float u = sc.dP[kb][i];                 // dP - D
      dd_acc += x;
      vP[e] = P;
      vx[e] = x;
      vu[e] = P * u;                              // P u
      vX[e] = fmaf(x, u, P * sc.dPa[kb][i]);      // P (dPa + ddS u)
      xs_acc += vX[e];
      pu_acc += vu[e];
    }
    const V8<T> oP = cvt8<T>(vP), ox = cvt8<T>(vx), ou = cvt8<T>(vu), oX = cvt8<T>(vX);
    ddr_acc = add_sum8<T>(ox, ddr_acc);
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const V8<T> tK = fr.trf(sa, 0, db);
      acc_a[db] = mma16<T>(fr.trf(sa, 2 * kTile, db), ou, acc_a[db]);
      acc_a[db] = mma16<T>(tK, oX, acc_a[db]);
      acc_s[db] = mma16<T>(tK, ou, acc_s[db]);
      acc_p[db] = mma16<T>(tK, oP, acc_p[db]);
      acc_o[db] = mma16<T>(fr.trf(sa, 3 * kTile, db), oP, acc_o[db]);
      acc_o[db] = mma16<T>(fr.trf(sa, kTile, db), ox, acc_o[db]);
    }
  };
  auto slot = [&](int kt) { return lds_kv + (uint32_t)(((uint32_t)kt % NST) * kStage); };
  // Waits for tile `need` and makes every wave's copy visible; `hi` is the last
  // tile issued (tiles after `need`, at most NST - 2, may still be in flight).
  auto advance = [&](int need) {
    const int ahead = hi - need;
    if (ahead >= 2)
      wait_vmem_le<2 * G::kLoads>();
    else if (ahead == 1)
      wait_vmem_le<G::kLoads>();
    else
      wait_vmem_le<0>();
    __syncthreads();
  };

  // Full tiles [0, nfull): visible to every query of the workgroup and inside
  // nk, so no mask. Pipelined: the scores of tile t + 1 are formed in the step
  // that finishes tile t, so each wave has independent matrix work to issue
  // beside its element-wise work. Buffers alternate, the loop being unrolled
  // by two.
  int full = p.nk / BK;
  if (CAUSAL) full = min(full, max(0, qb * BQ + p.coff + 1) / BK);
  const int nfull = __builtin_amdgcn_readfirstlane(min(full, nkt));
  auto step = [&](int t, Scores& cur, Scores& nxt, auto next_tag) {
    constexpr bool NEXT = decltype(next_tag)::value;
    advance(NEXT ? t + 1 : t);
    if (hi + 1 < nkt) issue(++hi);
    if constexpr (NEXT) scores(slot(t + 1), nxt);
    finish(slot(t), cur, 0, std::false_type{});
  };

  int t = 0;
  if (!PIPE) {
    for (; t < nfull; ++t) {
      advance(t);
      if (hi + 1 < nkt) issue(++hi);
      Scores A;
      scores(slot(t), A);
      finish(slot(t), A, 0, std::false_type{});
    }
  } else if (nfull > 0) {
    Scores A, B;
    advance(0);
    scores(slot(0), A);
    for (; t + 2 < nfull; t += 2) {
      step(t, A, B, std::true_type{});
      step(t + 1, B, A, std::true_type{});
    }
    if (t + 1 < nfull) {
      step(t, A, B, std::true_type{});
      step(t + 1, B, A, std::false_type{});
      t += 2;
    } else {
      step(t, A, B, std::false_type{});
      t += 1;
    }
  }
  // Diagonal and ragged tiles, one per step, masked; only waves with work.
  for (; t < nkt; ++t) {
    advance(t);
    if (hi + 1 < nkt) issue(++hi);
    if (t < wkt) {
      Scores sc;
      scores(slot(t), sc);
      const int klim = min(p.nk - 1, CAUSAL ? qi + p.coff : p.nk - 1) - t * BK;  // last visible key, tile-relative
      finish(slot(t), sc, klim, std::true_type{});
    }
  }

  const float dD = group4_sum(dd_acc);
  // ddO = acc_o - dD O, with dD summed over the T-rounded x that acc_o took
  // (see above).
  const float dDo = group4_sum(ddr_acc);
  // A row that sees exactly one key (see above).
  const bool one_key = (CAUSAL ? min(p.nk, qi + p.coff + 1) : p.nk) == 1;
  // c = D dD + B from the unrounded per-pair sums (see above).
  const float c = group4_sum(xs_acc) - dD * group4_sum(pu_acc);
  // ddO = acc_o - dD O, from this lane's four columns of each 16-column block
  // (16 db + 4 g + i).
  f32x4 y[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    const int d = 16 * db + 4 * g;
    const V4<T> o4 = *reinterpret_cast<const V4<T>*>(p.o + roff + d);
#pragma unroll
    for (int i = 0; i < 4; ++i) y[db][i] = acc_o[db][i] - dDo * (float)o4[i];
  }
  const float Bi = c - Di * dD;
  if (qvalid) {
    if (g == 0) {
      p.delta[sbase + qi] = Di;
      p.ddelta[sbase + qi] = dD;
      p.bstat[sbase + qi] = Bi;
    }
    T* dq2 = p.dq2 + roff;
    T* ddo = p.ddo + roff;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const int d = 16 * db + 4 * g;  // this lane's four output columns
      f32x4 x;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        x[i] = one_key ? 0.f : scale * (acc_a[db][i] - dD * acc_s[db][i] - c * acc_p[db][i]);
      *reinterpret_cast<V4<T>*>(dq2 + d) = cvt4<T>(x);
      *reinterpret_cast<V4<T>*>(ddo + d) = cvt4<T>(y[db]);
    }
  }
}

}  // namespace

template <typename T, int D, bool CAUSAL>
hipError_t launch_bwdbwd_stage1_fused(const BwdBwdParams<T>& p, hipStream_t stream) {
  const int nqb = (p.nq + kQ * kWaves - 1) / (kQ * kWaves);
  const int npairs = p.batch * p.heads;
  const int chunk = grid_chunk(npairs, nqb, resident_workgroups(D <= 128 ? 2 : 1));
  const dim3 grid(nqb * npairs);
  int e2;
  if (std::is_same_v<T, __bf16> && std::frexp(p.scale, &e2) == 0.5f)  // scale = 2^(e2 - 1)
    hipLaunchKernelGGL((bwdbwd_q_fused_kernel<T, D, CAUSAL, std::is_same_v<T, __bf16>>), grid, dim3(kThreads), 0,
                       stream, p, chunk);
  else
    hipLaunchKernelGGL((bwdbwd_q_fused_kernel<T, D, CAUSAL, false>), grid, dim3(kThreads), 0, stream, p, chunk);
  return hipGetLastError();
}

#define FHOG_INST(T, D, C) \
  template hipError_t launch_bwdbwd_stage1_fused<T, D, C>(const BwdBwdParams<T>&, hipStream_t);
FHOG_INST(__bf16, 64, true)
FHOG_INST(__bf16, 64, false)
FHOG_INST(_Float16, 64, true)
FHOG_INST(_Float16, 64, false)
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
