// Stage 1 of the Flash-HOG double backward (passes 1-3 in one sweep over the
// keys) for 2-byte types at D = 64: 32 queries per wave on the 32x32x16
// matrix instruction, one wave per SIMD, software-pipelined three tiles deep.
// The math and outputs are those of fhog_bwdbwd_fused.hip (which serves
// D = 128 and 256): with u = dP - D, x = P ddS, X = P (dPa + ddS u),
//   dQ2 = scale (sum_j P u ddK + sum_j X K - dD sum_j P u K - c sum_j P K),
//   ddO = sum_j P ddV + sum_j x V - dD' O,     c = D dD + B,
//   c = sum_j X - dD sum_j P u,  B = c - D dD,
// summed per pair in fp32 (flash_hog/_jax_refs/jax_impl.py:273-336, the pass
// split of flash_hog/jax/_pallas_gpu_kernel.py:149-278).
//
// Why this shape. A 16-query wave (the fused kernel) reads every key-side
// tile twice from LDS per 16 queries and issues a 16x16x32 instruction per
// 8192 multiply-adds; two such waves share a SIMD so that one wave's vector
// work overlaps the other's matrix work, and the matrix pipe stays about 43 %
// busy. With 32 queries per wave each LDS fragment serves twice the pairs and
// each matrix instruction does twice the work, but the four 32 x 64
// accumulators, two score sets and the resident operands need about 420
// registers, i.e. one wave per SIMD. A lone wave keeps the pipe fed only if
// its own instruction stream interleaves matrix, vector and LDS work, so each
// step of the loop mixes three tiles: the output products of tile t - 1, the
// element-wise step of tile t and the score products of tile t + 1, all
// independent of one another. (A loop of 44 such matrix instructions, 200
// vector and 48 LDS instructions and a barrier runs at 37.5 cycles per
// matrix instruction at one wave per SIMD: 85 % of the pipe.)
//
// Layouts (32x32x16, see fhog_device.h): score tiles are transposed,
// S^T = K Q^T, so lane n of a wave holds query q0 + n and register r key
// 8 (r / 4) + 4 g + r % 4 of the tile; a tile's registers 8 s .. 8 s + 7,
// converted to T, are the B operand of an output product over keys
// 16 s + 8 (e / 4) + 4 g + e % 4, whose A operand is the key-side tile read
// transposed in that order (SwzFrags::trf).
#include <cmath>
#include <type_traits>

#include "fhog_device.h"
#include "fhog_params.h"
#include "fhog_q32_loop.inc"

namespace fhog {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;

template <typename T, bool CAUSAL, bool PRE>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
bwdbwd_q32_kernel(BwdBwdParams<T> p, int chunk) {
  constexpr int D = 64;
  typedef SwzTile<T, D> G;
  constexpr int KS = D / 16;       // 16-deep steps over the head dim
  constexpr int DT = D / 32;       // 32-wide output column blocks
  constexpr int BQ = 32 * kWaves;  // queries per workgroup
  constexpr int BK = 32;           // keys per streamed tile
  // Ring: in a pipelined step tiles t - 1 (output products), t (whose
  // output products come next step) and t + 1 (score products) are in use
  // and tiles t + 2 .. t + 6 are in flight.
  constexpr int NST = 8;
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

  // Keys [0, kend) are visible to some query of the workgroup. Every wave
  // sweeps all of them (the sweep's barriers and LDS DMAs are shared); a wave
  // whose queries see none of a tile's keys masks all of its pairs.
  int kend = p.nk;
  if (CAUSAL) kend = min(kend, qb * BQ + BQ + p.coff);
  // (uniform; the sweep's branches depend only on such values)
  const int nkt = __builtin_amdgcn_readfirstlane(kend > 0 ? (kend + BK - 1) / BK : 0);

  SwzFrags<T, D> fr;
  fr.init(lane);
  // The transposed reads' second address is the first with bit 4 flipped
  // (SwzFrags::trf); ring stages are 32-byte aligned, so the flip can be
  // applied to the per-lane offset.
  const uint32_t ta0 = fr.tr[0], ta1 = fr.tr[1], tb0 = fr.tr[0] ^ 16u, tb1 = fr.tr[1] ^ 16u;

  // Wave w streams key-side tensor w (K, V, ddK, ddV) into the ring.
  const T* gnext = (wave == 0 ? p.k : wave == 1 ? p.v : wave == 2 ? p.ddk : p.ddv) + kbase;
  const uint32_t row_bytes = (uint32_t)(rsk * (long)sizeof(T));
  TileDma<T, D> dma, part;
  dma.init(row_bytes, BK, lane);
  // A ragged key tail can only be the last streamed tile; its loads repeat
  // row nk - 1 for the missing rows.
  const bool ragged = p.nk % BK != 0 && nkt == (p.nk + BK - 1) / BK;
  const int rag = ragged ? nkt - 1 : -1;
  part.init(row_bytes, ragged ? p.nk - (nkt - 1) * BK : BK, lane);
  const uint32_t lds_kv = lds_base_u32(s_kv);
  const uint32_t lds_wave = lds_kv + wave * kTile;
  const unsigned long gstep = (unsigned long)BK * (unsigned long)row_bytes;
  // The ring's first tiles (0 .. 4); the sweep issues the rest, tile t + 6 at
  // step t, into the stage tile t - 2 left. Tiles 0 and 1 go first, then the
  // query-side loads in one batch, then tiles 2 .. 4 once the query side has
  // been used: the compiler does not count the LDS DMAs (they are inline
  // assembly), so its waits for the query side also wait for every DMA
  // issued before them, and tiles issued later stream in while the sweep
  // starts.
  int hi = -1;
  auto issue_tile = [&]() {
    ++hi;
    const uint32_t dst = lds_wave + (uint32_t)(hi * kStage);
    if (hi == rag)
      part.issue(dst, gnext);
    else
      dma.issue(dst, gnext);
    gnext += BK * rsk;
  };
#pragma unroll
  for (int i = 0; i < 2; ++i)
    if (i < nkt) issue_tile();

  // Query-side operands (B of the score products), O for D_i = <O_i, dO_i>
  // and the logsumexp. A lane past the last query loads the last query's row:
  // its own results are never stored, and a matrix product column or row sum
  // of one query never mixes in another's, so finite values are all it
  // needs; loading unconditionally keeps the batch free of waits.
  V8<T> qf[KS], ddqf[KS], dof[KS], of[KS];
  const long roff = qbase + (long)min(qi, p.nq - 1) * rs;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const long off = roff + 16 * ks + 8 * g;
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
  const float Di = xgroup_sum(dpart);
  const float nD = -Di;
  const float nL2 = -lse * kLog2e;
  // O once more, in the accumulator layout, for the epilogue's
  // ddO = sum - dD' O (register 4 a + i of column block dt holds column
  // 32 dt + 8 a + 4 g + i); these loads land during the sweep.
  V4<T> oe[DT][4];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int a = 0; a < 4; ++a) oe[dt][a] = *reinterpret_cast<const V4<T>*>(p.o + roff + 32 * dt + 8 * a + 4 * g);
  // Everything the sweep takes from the query side is final before tiles
  // 2 .. 4 are issued (the empty statement pins that order), so no wait the
  // compiler places for it can count those DMAs.
  asm volatile("" ::"v"(qf[0]), "v"(qf[1]), "v"(qf[2]), "v"(qf[3]), "v"(ddqf[0]), "v"(ddqf[1]), "v"(ddqf[2]),
               "v"(ddqf[3]), "v"(dof[0]), "v"(dof[1]), "v"(dof[2]), "v"(dof[3]), "v"(nD), "v"(nL2));
#pragma unroll
  for (int i = 2; i < NST - 3; ++i)
    if (i < nkt) issue_tile();
  // No wait here: the sweep's DMA waits count the newest loads, and every
  // load above is older than tiles 2 .. 4.

  f32x16 acc_a[DT], acc_s[DT], acc_p[DT], acc_o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc_a[dt] = acc_s[dt] = acc_p[dt] = acc_o[dt] = zero16();
  float dd_acc = 0.f;   // dD = sum P ddS over this lane's keys
  // every row of ddm: the same sum over P ddS rounded to T, as the ddO
  // products take it (a matrix product with a ones operand)
  f32x16 ddm = zero16();
  const V8<T> ones = ones8<T>();
  float xs_acc = 0.f;   // sum X over this lane's keys
  float pu_acc = 0.f;   // sum P u over this lane's keys

  // Full tiles [0, nfull) are visible to every query of the workgroup and
  // inside nk; the element-wise step of a later tile masks keys past klim.
  int full = p.nk / BK;
  if (CAUSAL) full = min(full, max(0, qb * BQ + p.coff + 1) / BK);
  const int nfull = __builtin_amdgcn_readfirstlane(min(full, nkt));
  // last visible key of this lane's query, less 4 g (the key of accumulator
  // register r is 8 (r / 4) + 4 g + r % 4 of its tile)
  const int klb = min(p.nk - 1, CAUSAL ? qi + p.coff : p.nk - 1) - 4 * g;

  if (nkt > 0) {
#define FHOG_Q32_ARGS(LOOP)                                                                                 \
  asm volatile(LOOP                                                                                         \
               : [aa0] "+a"(acc_a[0]), [aa1] "+a"(acc_a[1]), [as0] "+a"(acc_s[0]), [as1] "+a"(acc_s[1]),   \
                 [ap0] "+a"(acc_p[0]), [ap1] "+a"(acc_p[1]), [ao0] "+a"(acc_o[0]), [ao1] "+a"(acc_o[1]),   \
                 [dd] "+v"(dd_acc), [ddm] "+a"(ddm), [xs] "+v"(xs_acc), [pu] "+v"(pu_acc)                  \
               : [q0] "a"(qf[0]), [q1] "a"(qf[1]), [q2] "a"(qf[2]), [q3] "a"(qf[3]), [dq0] "a"(ddqf[0]),   \
                 [dq1] "a"(ddqf[1]), [dq2] "a"(ddqf[2]), [dq3] "a"(ddqf[3]), [do0] "a"(dof[0]),            \
                 [do1] "a"(dof[1]), [do2] "a"(dof[2]), [do3] "a"(dof[3]), [nl2] "v"(nL2), [nd] "v"(nD),     \
                 [ones] "v"(ones),                                                                         \
                 [ro0] "v"(fr.row[0]), [ro1] "v"(fr.row[1]), [ro2] "v"(fr.row[2]), [ro3] "v"(fr.row[3]),   \
                 [ta0] "v"(ta0), [ta1] "v"(ta1), [tb0] "v"(tb0), [tb1] "v"(tb1), [vo0] "v"(dma.voff[0]),   \
                 [vo1] "v"(dma.voff[1]), [vo2] "v"(dma.voff[2]), [vo3] "v"(dma.voff[3]),                   \
                 [vp0] "v"(part.voff[0]), [vp1] "v"(part.voff[1]), [vp2] "v"(part.voff[2]),                \
                 [vp3] "v"(part.voff[3]), [klb] "v"(klb), [gptr] "s"(gnext), [gstep] "s"(gstep),           \
                 [hi0] "s"(hi), [ldskv] "s"(lds_kv), [ldsw] "s"(lds_wave), [nkt] "s"(nkt),                 \
                 [nfull] "s"(nfull), [rag] "s"(rag), [c2] "s"(c2), [scl] "s"(scale)                        \
               : FHOG_Q32_CLOBBERS)
    if constexpr (std::is_same_v<T, __bf16> && PRE)
      FHOG_Q32_ARGS(FHOG_Q32_LOOP_BF16_PRE);
    else if constexpr (std::is_same_v<T, __bf16>)
      FHOG_Q32_ARGS(FHOG_Q32_LOOP_BF16);
    else
      FHOG_Q32_ARGS(FHOG_Q32_LOOP_F16);
#undef FHOG_Q32_ARGS
  }

  const float dD = xgroup_sum(dd_acc);
  const float dDo = ddm[0];
  const bool one_key = (CAUSAL ? min(p.nk, qi + p.coff + 1) : p.nk) == 1;
  const float c = xgroup_sum(xs_acc) - dD * xgroup_sum(pu_acc);
  const float Bi = c - Di * dD;
  if (qvalid) {
    if (g == 0) {
      p.delta[sbase + qi] = Di;
      p.ddelta[sbase + qi] = dD;
      p.bstat[sbase + qi] = Bi;
    }
    T* dq2 = p.dq2 + roff;
    T* ddo = p.ddo + roff;
    // accumulator register 4 a + i of column block dt holds column
    // 32 dt + 8 a + 4 g + i of this lane's query
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d = 32 * dt + 8 * a + 4 * g;
        const V4<T> ov = oe[dt][a];
        f32x4 x, y;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 4 * a + i;
          x[i] = one_key ? 0.f : scale * (acc_a[dt][r] - dD * acc_s[dt][r] - c * acc_p[dt][r]);
          y[i] = acc_o[dt][r] - dDo * (float)ov[i];
        }
        *reinterpret_cast<V4<T>*>(dq2 + d) = cvt4<T>(x);
        *reinterpret_cast<V4<T>*>(ddo + d) = cvt4<T>(y);
      }
  }
}

}  // namespace

template <typename T, bool CAUSAL>
hipError_t launch_bwdbwd_stage1_q32(const BwdBwdParams<T>& p, hipStream_t stream) {
  const int nqb = (p.nq + 32 * kWaves - 1) / (32 * kWaves);
  const int npairs = p.batch * p.heads;
  const int chunk = grid_chunk(npairs, nqb, resident_workgroups(1));
  const dim3 grid(nqb * npairs);
  int e2;
  if (std::is_same_v<T, __bf16> && std::frexp(p.scale, &e2) == 0.5f)  // scale = 2^(e2 - 1)
    hipLaunchKernelGGL((bwdbwd_q32_kernel<T, CAUSAL, std::is_same_v<T, __bf16>>), grid, dim3(kThreads), 0, stream, p,
                       chunk);
  else
    hipLaunchKernelGGL((bwdbwd_q32_kernel<T, CAUSAL, false>), grid, dim3(kThreads), 0, stream, p, chunk);
  return hipGetLastError();
}

#define FHOG_INST(T, C) template hipError_t launch_bwdbwd_stage1_q32<T, C>(const BwdBwdParams<T>&, hipStream_t);
FHOG_INST(__bf16, true)
FHOG_INST(__bf16, false)
FHOG_INST(_Float16, true)
FHOG_INST(_Float16, false)
#undef FHOG_INST

}  // namespace fhog
