// Query-tiled kernel of the first-order attention backward (dQ and
// D = rowsum(O dO)) for 2-byte types at D = 64: 64 queries per wave at one
// wave per SIMD, the key sweep generated as inline assembly
// (gen_bwd_q64_loop.py -> fhog_bwd_q64_loop.inc). It computes what
// bwd_q_kernel (fhog_bwd.hip) computes, replacing part of the cuDNN backward
// the reference calls through flash_hog/jax/_attention_impl.py:242-261
// (equations of flash_hog/_jax_refs/jax_impl.py:142-191):
//   P = exp2(S scale log2 e - L log2 e), u = dP - D,  dQ = scale sum_k (P u) K,
// a pair (query, key) entering iff key <= query + coff (causal) and key < nk.
//
// Why this shape. bwd_q_kernel holds 32 queries per wave at two waves per
// SIMD and keeps the matrix pipe about 32 % busy. Here one wave holds 64
// queries (two halves of 32 with their own resident Q and dO, score tiles
// and dQ accumulators), so every key-side LDS fragment it reads serves twice
// the pairs, and the generated sweep interleaves the output products of tile
// t - 1, the element-wise step of tile t and the score products of tile
// t + 1. Score tiles are transposed (lane = query), so L and D are per-lane
// scalars: the exponent takes -L log2 e as an fma operand and the dP chains
// start at a 16-register tuple of -D.
//
// A workgroup owns 256 queries of one (batch, head) pair and streams 32-key
// tiles of K (wave 0) and V (wave 1) of the head's key/value head through an
// 8-stage LDS ring of 8 KiB stages. Causal query blocks are taken in mirror
// pairs (the longest block, then the shortest) when the grid outnumbers the
// CUs.
#include <cmath>
#include <cstdint>

#include "fhog_bwd_q64_loop.inc"
#include "fhog_device.h"
#include "fhog_params.h"

namespace fhog {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;

__device__ __forceinline__ uint32_t uni(uint32_t x) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)x); }
__device__ __forceinline__ float uni(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, x)));
}
__device__ __forceinline__ uint64_t uni(uint64_t x) {
  return (uint64_t)uni((uint32_t)x) | ((uint64_t)uni((uint32_t)(x >> 32)) << 32);
}
__device__ __forceinline__ const void* uni(const void* x) { return (const void*)(uintptr_t)uni((uint64_t)(uintptr_t)x); }

template <typename T, bool CAUSAL>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
bwd_q64_kernel(BwdParams<T> p, int pairs, int chunk) {
  constexpr int D = 64;
  typedef SwzTile<T, D> G;
  constexpr int KS = D / 16;
  constexpr int DT = D / 32;
  constexpr int QW = 64;            // queries per wave
  constexpr int BQB = QW * kWaves;  // queries per workgroup
  constexpr int BK = 32;            // keys per streamed tile
  constexpr int NST = 8;
  constexpr int kTile = G::kElems * (int)sizeof(T);
  constexpr int kStage = 2 * kTile;  // K, V
  static_assert(kTile == 4096, "the generated sweep assumes 4 KiB tiles");
  // the ring, then per wave the staged query side: Q, dO and O of its two
  // halves (six tiles; 160 KiB in all)
  __shared__ __attribute__((aligned(1024))) char s_kv[NST * kStage + kWaves * 6 * kTile];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 31, g = lane >> 5;
  const int nbh = p.batch * p.heads;
  const int nqb = (p.nq + BQB - 1) / BQB;
  const GridSlot slot = grid_slot(blockIdx.x, nbh, pairs ? (nqb + 1) / 2 : nqb, chunk);
  const int bh = slot.pair;
  const BlockPair bp = block_pair(slot.rank, nqb, pairs);
  const float scale = p.scale;

  for (int blk = 0; blk < bp.count; ++blk) {
    const int rank = blk == 0 ? bp.first : bp.second;
    const int qb = CAUSAL ? nqb - 1 - rank : rank;  // causal: rank 0 is the block with the longest rows
    if (blk > 0) __syncthreads();  // every wave is done with the previous block's ring
    const int b = bh / p.heads, h = bh % p.heads;
    const int hk = h / (p.heads / p.kv_heads);
    const long rs = (long)p.heads * D;      // query-side row stride
    const long rsk = (long)p.kv_heads * D;  // key-side row stride
    const long qbase = ((long)b * p.nq * p.heads + h) * D;
    const long kbase = ((long)b * p.nk * p.kv_heads + hk) * D;
    const long sbase = (long)bh * p.nq;
    const int q0 = qb * BQB + wave * QW;  // half h holds queries q0 + 32 h + n
    // Keys [0, kend) are visible to some query of the block; every wave sweeps
    // all of them (the sweep's barriers and DMAs are shared).
    int kend = p.nk;
    if (CAUSAL) kend = min(kend, qb * BQB + BQB + p.coff);
    const int ntot = __builtin_amdgcn_readfirstlane(kend > 0 ? (kend + BK - 1) / BK : 0);

    f32x16 acc[2][DT];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc[hh][dt] = zero16();

    float Di[2] = {0.f, 0.f};
    if (ntot == 0) {
      // a block that sees no key: dQ = 0, and D is still written
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const long roff = qbase + (long)min(q0 + 32 * hh + n, p.nq - 1) * rs;
        float dpart = 0.f;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const long off = roff + 16 * ks + 8 * g;
          dpart = dot8<T>(*reinterpret_cast<const V8<T>*>(p.o + off), *reinterpret_cast<const V8<T>*>(p.dout + off),
                          dpart);
        }
        Di[hh] = xgroup_sum(dpart);
      }
    } else {
      SwzFrags<T, D> fr;
      fr.init(lane);
      const uint32_t ta0 = fr.tr[0], ta1 = fr.tr[1], tb0 = fr.tr[0] ^ 16u, tb1 = fr.tr[1] ^ 16u;
      const uint32_t lds_k = lds_base_u32(s_kv);
      const bool tens = wave < 2;

      // Streams and their per-lane offsets. The ragged last key tile (if
      // nk % 32 != 0) repeats row nk - 1 for its missing rows.
      const int nkt_all = (p.nk + BK - 1) / BK;
      const int rag_rows = p.nk - (nkt_all - 1) * BK;
      const uint32_t ragk0 = rag_rows < BK ? (uint32_t)((nkt_all - 1) * BK) : 0xffffffffu;
      const uint32_t row_bytes = (uint32_t)(rsk * (long)sizeof(T));
      TileDma<T, D> dma, part;
      dma.init(row_bytes, BK, lane);
      part.init(row_bytes, rag_rows, lane);
      const char* ptr = reinterpret_cast<const char*>((wave == 0 ? p.k : p.v) + kbase);
      const uint64_t gstep = (uint64_t)BK * row_bytes;
      const uint32_t ldsw = wave == 0 ? 0u : wave == 1 ? (uint32_t)kTile : (uint32_t)FHOG_BQ64_WAVE_NONE;

      // DMA cursor: the next tile to issue starts at key dk0
      uint32_t dk0 = 0;
      int hi = -1;
      auto issue_tile = [&]() {
        ++hi;
        const uint32_t dst = lds_k + (uint32_t)((hi % NST) * kStage) + ldsw;
        const uint32_t* off = dk0 == ragk0 ? part.voff : dma.voff;
        if (tens) {
          dma16s(ptr, off[0], dst);
#pragma unroll
          for (int j = 1; j < 4; ++j) dma16s_next(ptr, off[j], dst + 1024u * j);
        }
        dk0 += BK;
        ptr += gstep;
      };
      // Tiles 0 and 1 first, then the query-side loads, then tiles 2 .. 4
      // once those have been used (the compiler's waits for its loads also
      // wait for every DMA issued before them; the sweep's waits count DMAs
      // and are only made stricter by older loads).
#pragma unroll
      for (int i = 0; i < 2; ++i)
        if (i < ntot) issue_tile();
      // The query side: Q and dO (B operands of the score products) and
      // D = rowsum(O dO), for each half (with dot8, as bwd_q_kernel sums
      // it). The rows move HBM -> LDS eight
      // 128-byte rows per instruction (in the operand layout a load touches
      // 32 rows) into this wave's staging tiles, and are read back in the
      // operand layout; rows past the last query repeat row nq - 1 (their
      // results are never stored).
      const uint32_t lds_qs = uni(lds_k + (uint32_t)(NST * kStage + wave * 6 * kTile));
      const uint32_t row_bytes_q = (uint32_t)(rs * (long)sizeof(T));
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int q0c = min(q0 + 32 * hh, p.nq - 1);
        TileDma<T, D> qd;
        qd.init(row_bytes_q, p.nq - q0c, lane);
        const long off = qbase + (long)q0c * rs;
        qd.issue(lds_qs + (uint32_t)(hh * kTile), uni((const void*)(p.q + off)));
        qd.issue(lds_qs + (uint32_t)((2 + hh) * kTile), uni((const void*)(p.dout + off)));
        qd.issue(lds_qs + (uint32_t)((4 + hh) * kTile), uni((const void*)(p.o + off)));
      }
      // -L log2 e per half (a row that sees no key has L = +inf: P = 0)
      float nl[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int qi = q0 + 32 * hh + n;
        nl[hh] = qi < p.nq ? -p.lse[sbase + qi] * kLog2e : 0.f;
      }
      asm volatile("s_waitcnt vmcnt(0)" : "+v"(nl[0]), "+v"(nl[1])::"memory");
      V8<T> qf[2][KS], dof[2][KS];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        float dpart = 0.f;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          qf[hh][ks] = fr.rowf(lds_qs, hh * kTile, ks);
          dof[hh][ks] = fr.rowf(lds_qs, (2 + hh) * kTile, ks);
          dpart = dot8<T>(fr.rowf(lds_qs, (4 + hh) * kTile, ks), dof[hh][ks], dpart);
        }
        Di[hh] = xgroup_sum(dpart);
      }

#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        asm volatile("" ::"v"(qf[0][ks]), "v"(qf[1][ks]), "v"(dof[0][ks]), "v"(dof[1][ks]), "v"(Di[0]), "v"(Di[1]),
                     "v"(nl[0]), "v"(nl[1]));
      asm volatile("" ::: "memory");
#pragma unroll
      for (int i = 2; i < NST - 3; ++i)
        if (i < ntot) issue_tile();

      // -D per half, and the masks' key bounds
      const float c2 = scale * kLog2e;
      float nd[2];
      int klb[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int qi = q0 + 32 * hh + n;
        nd[hh] = -Di[hh];
        // the lane's last visible key, less 4 g: the key of accumulator
        // register r is 8 (r / 4) + 4 g + r % 4 of its tile
        klb[hh] = min(p.nk - 1, CAUSAL ? qi + p.coff : p.nk - 1) - 4 * g;
      }
      // Full tiles [0, nfull) are visible to every query of the block and
      // inside nk; later tiles take the masked element-wise step.
      int full = p.nk / BK;
      if (CAUSAL) full = min(full, max(0, qb * BQB + p.coff + 1) / BK);
      const int nfull = __builtin_amdgcn_readfirstlane(min(full, ntot));
      // steady steps (no branches in their DMA) need tile t + 6 to be a full tile
      const int nsd = __builtin_amdgcn_readfirstlane(ntot - (rag_rows < BK && ntot == nkt_all ? 1 : 0));
      const uint32_t u_ldsk = uni(lds_k), u_ldsw = uni(ldsw), u_ragk0 = uni(ragk0);
      uint32_t r_hi = uni((uint32_t)hi), r_dgi = 0, r_dq0 = uni(dk0), r_eq0 = 0;
      const float u_c2 = uni(c2);
      const uint32_t gstep_lo = uni((uint32_t)gstep), gstep_hi = uni((uint32_t)(gstep >> 32));
      uint64_t r_p0 = uni((uint64_t)(uintptr_t)ptr);

#define FHOG_BQ64_ARGS(LOOP)                                                                                  \
  asm volatile(LOOP                                                                                           \
               : [aq00] "+a"(acc[0][0]), [aq01] "+a"(acc[0][1]), [aq10] "+a"(acc[1][0]),                   \
                 [aq11] "+a"(acc[1][1]), FHOG_BQ64_BOUND(r_hi, r_dgi, r_dq0, r_eq0, r_p0)                    \
               : [q00] "a"(qf[0][0]), [q01] "a"(qf[0][1]), [q02] "a"(qf[0][2]), [q03] "a"(qf[0][3]),       \
                 [q10] "a"(qf[1][0]), [q11] "a"(qf[1][1]), [q12] "a"(qf[1][2]), [q13] "a"(qf[1][3]),       \
                 [o00] "a"(dof[0][0]), [o01] "a"(dof[0][1]), [o02] "a"(dof[0][2]), [o03] "a"(dof[0][3]),   \
                 [o10] "a"(dof[1][0]), [o11] "a"(dof[1][1]), [o12] "a"(dof[1][2]), [o13] "a"(dof[1][3]),   \
                 [ro0] "v"(fr.row[0]), [ro1] "v"(fr.row[1]), [ro2] "v"(fr.row[2]), [ro3] "v"(fr.row[3]),   \
                 [ta0] "v"(ta0), [ta1] "v"(ta1), [tb0] "v"(tb0), [tb1] "v"(tb1), [vo0] "v"(dma.voff[0]),   \
                 [vo1] "v"(dma.voff[1]), [vo2] "v"(dma.voff[2]), [vo3] "v"(dma.voff[3]),                   \
                 [vp0] "v"(part.voff[0]), [vp1] "v"(part.voff[1]), [vp2] "v"(part.voff[2]),                \
                 [vp3] "v"(part.voff[3]), [nl0] "v"(nl[0]), [nl1] "v"(nl[1]), [nd0] "v"(nd[0]),             \
                 [nd1] "v"(nd[1]), [klb0] "v"(klb[0]), [klb1] "v"(klb[1]), [ldsk] "s"(u_ldsk),              \
                 [ldsw] "s"(u_ldsw), [ntot] "s"(ntot), [nfull] "s"(nfull), [nsd] "s"(nsd),                  \
                 [ragk0] "s"(u_ragk0), [c2] "s"(u_c2), [gstep_lo] "s"(gstep_lo), [gstep_hi] "s"(gstep_hi)   \
               : FHOG_BQ64_CLOBBERS)
      if constexpr (std::is_same_v<T, __bf16>)
        FHOG_BQ64_ARGS(FHOG_BQ64_LOOP_BF16);
      else
        FHOG_BQ64_ARGS(FHOG_BQ64_LOOP_F16);
#undef FHOG_BQ64_ARGS
      (void)r_dgi;
    }

    // dQ goes to HBM as whole 128-byte rows, eight rows per store
    // instruction, through an 8 KiB staging area per wave: wave w stages in
    // the ring stage of tile ntot - 8 + w, which no wave reads any more (every
    // wave has passed the barrier that waited for tile ntot - 1) and no DMA
    // writes. Rows are swizzled by query mod 8 so that neither the writes nor
    // the row reads conflict. (The lane index is made opaque here, so that
    // these addresses are formed after the sweep instead of being kept alive
    // across it.)
    int le = lane;
    asm volatile("" : "+v"(le));
    const int ne = le & 31, ge = le >> 5;
    const uint32_t stg = lds_base_u32(s_kv) + (uint32_t)(((uint32_t)(ntot + wave) & (NST - 1)) * kStage);
    // accumulator register 4 a + i of column block dt holds column
    // 32 dt + 8 a + 4 g + i of this lane's query (row 32 h + n of the stage)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int r = 32 * hh + ne;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          f32x4 x;
#pragma unroll
          for (int i = 0; i < 4; ++i) x[i] = acc[hh][dt][4 * a + i] * scale;
          const uint32_t off = (uint32_t)(r * 128 + 16 * phys_chunk<kSwzRows>(r, 4 * dt + a) + 8 * ge);
          *reinterpret_cast<__attribute__((address_space(3))) V4<T>*>((uintptr_t)(stg + off)) = cvt4<T>(x);
        }
      const int qi = q0 + r;
      if (ge == 0 && qi < p.nq) p.delta[sbase + qi] = Di[hh];
    }
    // lane l takes 16 bytes of row 8 i + l / 8 (chunk position l % 8, holding
    // logical chunk (l % 8) ^ (row mod 8))
    const int lc = (le & 7) ^ ((le >> 3) & 7);
    V8<T> rows[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      rows[i] = *reinterpret_cast<const __attribute__((address_space(3))) V8<T>*>(
          (uintptr_t)(stg + 1024u * i + 16u * (uint32_t)le));
    T* dst = p.dq + qbase + 8 * lc;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int qr = q0 + 8 * i + (le >> 3);
      if (qr < p.nq) *reinterpret_cast<V8<T>*>(dst + (long)qr * rs) = rows[i];
    }
  }
}

}  // namespace

template <typename T, bool CAUSAL>
hipError_t launch_bwd_q64(const BwdParams<T>& p, hipStream_t stream) {
  const int nqb = (p.nq + 64 * kWaves - 1) / (64 * kWaves);
  const int npairs = p.batch * p.heads;
  const int resident = resident_workgroups(1);
  const int pairs = block_pairing(CAUSAL, nqb, npairs, resident, 1);
  const int nranks = pairs ? (nqb + 1) / 2 : nqb;
  const int chunk = grid_chunk(npairs, nranks, resident);
  hipLaunchKernelGGL((bwd_q64_kernel<T, CAUSAL>), dim3(nranks * npairs), dim3(kThreads), 0, stream, p, pairs,
                     chunk);
  return hipGetLastError();
}

template hipError_t launch_bwd_q64<__bf16, true>(const BwdParams<__bf16>&, hipStream_t);
template hipError_t launch_bwd_q64<__bf16, false>(const BwdParams<__bf16>&, hipStream_t);
template hipError_t launch_bwd_q64<_Float16, true>(const BwdParams<_Float16>&, hipStream_t);
template hipError_t launch_bwd_q64<_Float16, false>(const BwdParams<_Float16>&, hipStream_t);

}  // namespace fhog
