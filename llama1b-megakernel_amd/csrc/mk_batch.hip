// mk_batch.hip — batched decode step of libmk.so for MI355X (gfx950): one
// persistent launch advances up to 32 independent sequences by one token.
//
// Same phases as the batch-1 kernel (mk_decode.hip) — per layer QKV (RMSNorm,
// projection, RoPE, K/V scatter at each sequence's own position), split-K GQA
// attention over each sequence's own KV length, O projection + residual,
// RMSNorm + gate/up + SwiGLU, down projection + residual; then final norm,
// tied lm_head and a greedy argmax per sequence — with these differences:
//
//   * projections are bf16 MFMA GEMMs (v_mfma_f32_16x16x32_bf16, fp32
//     accumulation): the tokens of the batch are the M dimension (one 16-row
//     tile for up to 16 sequences, two for up to 32), 16 weight rows the N
//     dimension. Each lane streams its B operand straight from HBM: 16 bytes
//     of one weight row per k-step (row n0 + lane%16, columns k + (lane/16)*8),
//     so every weight byte is loaded once per step, as at batch 1;
//   * phases with one 16-row tile per workgroup (QKV, O, down) split K over
//     the 4 waves and sum the 4 partial tiles through LDS in a fixed order;
//     phases with many tiles per workgroup (gate/up, lm_head) give each wave
//     whole tiles;
//   * the A operand (activations) comes from LDS where the input is normalised
//     (QKV, gate/up, lm_head: the staged [tokens][2048] matrix), or straight
//     from the exchange buffer in MFMA layout (O, down);
//   * hand-overs use arrival counters instead of sentinel data: every
//     activation matrix is read by every workgroup, so consumers read it with
//     ordinary loads that the XCD's L2 serves to its 32 CUs after the first
//     fetch. A producer workgroup stores its results (device scope), waits
//     for the stores to complete and adds one to its sub-counter (8 per
//     hand-over, on separate lines, so arrivals do not queue on one line); a
//     consumer polls the 8 sub-counters, then reads. A buffer is written once
//     per launch and read only after its counter is complete, and every
//     launch starts with invalidated caches, so no cached copy is stale;
//   * staged inputs go straight from memory into LDS (buffer loads to LDS),
//     leaving the registers to the weight stream;
//   * attention work items are (sequence, kv head, KV split), sized from all
//     sequences' lengths so the grid gets balanced work; the partials of a
//     (sequence, kv head) are merged by whichever workgroup finishes its last
//     split (an arrival counter), so no workgroup waits for another's
//     attention work.
#include <hip/hip_runtime.h>

#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "mk.h"
#include "mk_batch.h"
// The two-token-tile instantiations (batches 17..32) are compiled in a
// translation unit of their own, mk_batch_tile2.hip, which includes this file
// with MK_BATCH_TILE2 defined. There the thread index is opaque to the
// optimiser (tid() in mk_common.h): with less state kept live in registers
// that kernel ran 1% faster at batch 32; the one-tile kernel, compiled here
// with the plain index, ran 1.7% slower with it at batch 8.
#ifdef MK_BATCH_TILE2
#define MK_OPAQUE_TID 1
#endif
#include "mk_common.h"

// Tuning constants (values measured best on MI355X; the alternatives and their
// results are recorded with the design notes).
constexpr int BATT_DEPTH = 1;   // 128-row K/V groups an attention item keeps in flight ahead
constexpr int BGU_CH = 4;       // one tile: 1 KiB gate/up LDS copies per wave per poll round of the h1 wait
constexpr int BGU_CH_O = 8;     // ... of the attention-output wait (O phase)
constexpr int BGU_SKIP_O = 1;   // failed polls of that wait before its copies start
constexpr int BDN_RING = 4;     // down projection: weight/act units in flight per wave
constexpr int BDN_PRE = 4;      // of which issued before the act wait (weights only)

namespace {

using namespace mk;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int XS = H + 8;      // LDS row stride (bf16) of a staged activation matrix (+16 B against bank conflicts)
constexpr int RES_MAX = 64;    // residual columns per workgroup kept in LDS (H / 32 at the smallest grid)
constexpr int KQ = H / NWAVE;  // 512: the K range of one wave in the split-K phases over H
constexpr int KS = 16;         // k-steps (of 32 columns) in a weight unit of the LDS-operand phases
constexpr int DKS = 8;         // k-steps in a unit of the down projection (A operand in registers too)
constexpr int B_MIN_GRID = 32;
constexpr int C_EXIT = 0, C_ERR = 1, C_EPOCH = 2;   // control words (shared with the batch-1 layout)
constexpr int HO_QKV = 0, HO_ATT = 1, HO_H1 = 2, HO_ACT = 3, HO_H2 = 4;   // hand-overs of a layer

struct BParams {
  const uint16_t* w_qkv;
  const uint16_t* w_o;
  const uint16_t* w_gu;
  const uint16_t* w_d;
  const uint16_t* embed;
  const uint16_t* lm;   // the lm_head rows: embed, or its tiled copy
  int tiled;            // w_qkv, w_o, w_gu, w_d and lm are the tiled copies
  const uint16_t* g_final;
  const uint16_t* rope;
  uint16_t* kc[MK_MAX_LAYERS];
  uint16_t* vc[MK_MAX_LAYERS];
  const int32_t* tokens;
  const uint16_t* hidden_in;
  int32_t* pos;
  uint16_t* hidden_out;
  float* logits;
  int32_t* next_token;
  uint8_t* ws;
  uint8_t* xch;
  uint8_t* cnt;         // the two arrival-counter sets
  BatchLayout lay;
  int batch;
  int max_batch;
  int first_layer;
  int n_layers;
  int s_max;
  int rope_rows;
  int do_lm;
  uint32_t flags;
  unsigned long long timeout_ticks;
  unsigned long long* trace;
};

template <int MT>
struct BLds {
  __attribute__((aligned(16))) uint16_t xn[16 * MT][XS];        // staged activation (normalised in place)
  __attribute__((aligned(16))) uint16_t res[16 * MT][RES_MAX];  // raw columns [R0, R1) of the staged input
  f32x4 red[NWAVE][MT][64];                                     // split-K partial tiles
  __attribute__((aligned(16))) uint16_t q[GQA * HD + 2 * HD];    // attention: 4 q heads | fresh k | fresh v
  __attribute__((aligned(16))) uint16_t rope[16 * MT][2 * HD];   // each token's RoPE row: cos | sin
  AttnShared att;
  unsigned long long key[NWAVE][16 * MT];
  int pos[BATCH_MAX];
  int tok[BATCH_MAX];
  int ns[BATCH_MAX];
  int ng[BATCH_MAX];         // attention plan: 128-row groups per kv head of each sequence
  int cum[BATCH_MAX + 1];    // attention plan: first item of each sequence
  int flag;
  float ssq[NWAVE][16 * MT];   // QKV: each wave's sum of squares of every row over its K quarter
  // gate/up with one token tile: the last weight unit of each wave's tile,
  // copied from HBM while the workgroup waits for the attention output and
  // for h1 (k-step s of wave w at
  // gw[(w*KS + s)*64], lane l's 16 bytes at + l, the register unit's lane
  // order), and a 1 KiB area per wave that copies past it write (two tiles
  // leave no room in LDS for either)
  static constexpr int GW = MT == 1 ? NWAVE * KS * 64 : 1;
  u32x4 gw[GW];
  u32x4 gspare[GW > 1 ? NWAVE * 64 : 1];
};

struct BCtx {
  const BParams* p;
  Sync s;
  int G, w, B;
  bool prefill;     // MK_FLAG_PREFILL: every token uses sequence 0 of the caches
  __device__ __forceinline__ int cache_seq(int b) const { return prefill ? 0 : b; }
  uint8_t* hcnt;    // this launch's hand-over counters [layer][5][8 lines]
  uint32_t* acnt;   // this launch's attention-split counters [layer][M][8]
  uint32_t* dcnt;   // this launch's down-projection row-group counters [layer][DN_MAX]
  // 2-D down projection (batches above 16): workgroup w computes rows
  // [n*drpg, (n+1)*drpg), n = w / 4, over the K quarter w % 4 (needs grid % 4 == 0
  // and whole 16-row tiles per group)
  bool d2;
  int dng, drpg;
  bool dpair;       // every workgroup has at most 8 rows of the (1-D) down projection
  uint8_t* sset;    // this launch's sentinel-filled exchange set (qkv of every layer)
  uint32_t* cnt_other;   // the other counter set (the next launch's), zeroed by this one
  int cnt_words;
  __device__ __forceinline__ uint16_t* xb(int li, size_t off) const {
    return reinterpret_cast<uint16_t*>(p->xch + (size_t)li * p->lay.layer + off);
  }
  __device__ __forceinline__ uint16_t* sx(int li, size_t off) const {
    return reinterpret_cast<uint16_t*>(sset + (size_t)li * p->lay.sset_layer + off);
  }
  __device__ __forceinline__ float* part(int li, int b, int h, int sp) const {
    return reinterpret_cast<float*>(p->xch + p->lay.part_base + (size_t)li * p->lay.part_layer) +
           ((size_t)(b * NKV + h) * BATT_MAX_SPLIT + sp) * PART_FLOATS;
  }
  __device__ __forceinline__ float* dpart(int li) const {
    return reinterpret_cast<float*>(p->xch + p->lay.dpart_base + (size_t)li * p->lay.dpart_layer);
  }
  __device__ __forceinline__ uint32_t* ho(int li, int k) const {
    return reinterpret_cast<uint32_t*>(hcnt + ((size_t)li * N_HANDOVER + k) * N_SUB * CNT_LINE);
  }
};

// The kernel's parameter block (its one explicit argument, at offset 0 of the
// kernarg segment) and a uniform value, through opaque copies: the compiler
// can neither hoist loads or arithmetic on them out of a loop nor merge them
// with earlier ones (see tid() in mk_common.h).
__device__ __forceinline__ const BParams* opaque_params() {
  typedef const __attribute__((address_space(4))) BParams* KParamPtr;
  KParamPtr k = (KParamPtr)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(k));
  return (const BParams*)k;
}
__device__ __forceinline__ int opaque_s(int v) {
  asm volatile("" : "+s"(v));
  return v;
}

__device__ __forceinline__ int xk(int li, int ph) { return 5 * li + ph; }

// Integer reductions over the 64 lanes of a wave (every lane gets the result),
// and an inclusive prefix sum in lane order: DPP steps within each 16-lane row,
// then the four row results through v_readlane (a lane shuffle would be an LDS
// round trip per step).
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ uint32_t lane_u32(uint32_t v, int l) { return (uint32_t)__builtin_amdgcn_readlane((int)v, l); }
constexpr int DPP_SHR1 = 0x111, DPP_SHR2 = 0x112, DPP_SHR4 = 0x114, DPP_SHR8 = 0x118;   // row_shr:n (0 shifted in)
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
  v += dpp_u32<DPP_XOR1>(v);
  v += dpp_u32<DPP_XOR2>(v);
  v += dpp_u32<DPP_ROR4>(v);
  v += dpp_u32<DPP_ROR8>(v);   // every lane: the sum of its row
  return (lane_u32(v, 0) + lane_u32(v, 16)) + (lane_u32(v, 32) + lane_u32(v, 48));
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  auto mx = [](uint32_t a, uint32_t b) { return a > b ? a : b; };
  v = mx(v, dpp_u32<DPP_XOR1>(v));
  v = mx(v, dpp_u32<DPP_XOR2>(v));
  v = mx(v, dpp_u32<DPP_ROR4>(v));
  v = mx(v, dpp_u32<DPP_ROR8>(v));
  return mx(mx(lane_u32(v, 0), lane_u32(v, 16)), mx(lane_u32(v, 32), lane_u32(v, 48)));
}
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
  const int lane = lane_id();
  v += dpp_u32<DPP_SHR1>(v);
  v += dpp_u32<DPP_SHR2>(v);
  v += dpp_u32<DPP_SHR4>(v);
  v += dpp_u32<DPP_SHR8>(v);   // inclusive scan within each row
  const uint32_t r0 = lane_u32(v, 15), r1 = lane_u32(v, 31), r2 = lane_u32(v, 47);
  return v + (lane >= 16 ? r0 : 0u) + (lane >= 32 ? r1 : 0u) + (lane >= 48 ? r2 : 0u);
}

// ---------------------------------------------------------------------------
// Hand-overs
// ---------------------------------------------------------------------------

// The workgroup's results of a phase are complete: every thread's stores
// have finished, then one arrival is added to sub-counter `sub` of the hand-over.
__device__ __forceinline__ void arrive(uint32_t* ho, int sub) {
  wait_mem();
  lds_sync();
  if (tid() == 0)
    __hip_atomic_fetch_add(reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(ho) + (size_t)sub * CNT_LINE), 1u,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wait (one full wave) until sub-counter j of a hand-over holds per + (j < extra) arrivals.
__device__ __forceinline__ void wait_handover(const Sync& sy, const uint32_t* ho, int per, int extra) {
  const int lane = lane_id();
  const rsrc_t r = make_rsrc(ho, N_SUB * CNT_LINE);
  const uint32_t off = lane < N_SUB ? (uint32_t)(lane * CNT_LINE) : OOB;
  const uint32_t target = lane < N_SUB ? (uint32_t)(per + (lane < extra ? 1 : 0)) : 0u;
  const unsigned long long t0 = wall_clock64();
  for (int it = 1;; ++it) {
    const uint32_t v = ld_dev4(r, off);
    if (__all(v >= target)) return;
    if (wait_expired(sy, t0, it)) return;
    __builtin_amdgcn_s_sleep(1);
  }
}
// One weight unit (KS k-steps in load_w's lane layout) copied from HBM into
// LDS at dst (KS x 1 KiB: k-step s at dst + s*64, lane l's 16 bytes at + l), a
// few 1 KiB copies at a time, so that the copies fill the hand-over wait
// before the unit is used without one burst of them queueing ahead of the
// poll.
// (UnitCopyT<N>: the first N k-steps of such a unit, N x 1 KiB.)
template <int N>
struct UnitCopyT {
  rsrc_t r;
  uint32_t o, step;
  int next;   // k-steps issued (N: all, or no copy)
  __device__ __forceinline__ void init(rsrc_t rw, bool tiled, int row, int row_end, uint32_t row_bytes, int k0,
                                       bool on) {
    const int lane = lane_id();
    const int n = row + (lane & 15);
    if (tiled) {
      const uint32_t kb = row_bytes / 64u;
      o = (((uint32_t)n >> 4) * kb + ((uint32_t)k0 >> 5)) * 1024u + (uint32_t)(lane >> 4) * 256u + (uint32_t)(n & 15) * 16u;
      step = 1024u;
    } else {
      o = (uint32_t)n * row_bytes + (uint32_t)(k0 + (lane >> 4) * 8) * 2u;
      step = 64u;
    }
    if (n >= row_end) o = OOB;
    r = rw;
    next = on ? 0 : N;
  }
  // up to n more k-steps
  __device__ __forceinline__ void issue(int n, u32x4* dst) {
    const int end = min(N, next + n);
    for (; next < end; ++next)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)(dst + next * 64), 16, o + (uint32_t)next * step, 0, 0,
                                               AUX_NT);
  }
  // the rest, as exactly K copy instructions (a fixed count, so that a wait
  // for loads issued before them can count past them): k-steps already issued
  // go to `spare`, a 1 KiB area nobody reads, from an out-of-range offset
  // (no memory read)
  template <int K>
  __device__ __forceinline__ void issue_fixed(u32x4* dst, u32x4* spare) {
    const int nx = __builtin_amdgcn_readfirstlane(next);
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int ck = nx + k;
      const bool real = ck < N;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)(real ? dst + ck * 64 : spare), 16,
                                               real ? o + (uint32_t)ck * step : OOB, 0, 0, AUX_NT);
    }
    next = min(N, nx + K);
  }
};
using UnitCopy = UnitCopyT<KS>;

// The gate/up weights a wave copies to LDS ahead of the gate/up phase (one
// token tile, one weight tile per wave): u3, the tile's last unit, into gw;
// u2, the first half of its unit 2, into rows 8..15 of the staged matrix when
// the batch has at most 8 tokens (those rows are MFMA padding whose products
// are discarded; the h1 staging then leaves them alone). issue(n) takes u3's
// copies first.
struct GuCopy {
  UnitCopy u3;
  UnitCopyT<KS / 2> u2;
  u32x4* d3;
  u32x4* d2;
  bool half;   // u2 is live (workgroup-uniform)
  __device__ __forceinline__ void issue(int n, u32x4*) {
    const int before = u3.next;
    u3.issue(n, d3);
    u2.issue(n - (u3.next - before), d2);
  }
};

// wait_handover that issues `ch` more copies of `uc` after every poll that
// finds the hand-over incomplete (the next poll queues behind them).
template <class Copy>
__device__ __forceinline__ void wait_handover_copy(const Sync& sy, const uint32_t* ho, int per, int extra,
                                                   Copy& uc, int ch, u32x4* dst, int skip = 0) {
  const int lane = lane_id();
  const rsrc_t r = make_rsrc(ho, N_SUB * CNT_LINE);
  const uint32_t off = lane < N_SUB ? (uint32_t)(lane * CNT_LINE) : OOB;
  const uint32_t target = lane < N_SUB ? (uint32_t)(per + (lane < extra ? 1 : 0)) : 0u;
  const unsigned long long t0 = wall_clock64();
  for (int it = 1;; ++it) {
    const uint32_t v = ld_dev4(r, off);
    if (__all(v >= target)) return;
    if (wait_expired(sy, t0, it)) return;
    if (it > skip) uc.issue(ch, dst);
    __builtin_amdgcn_s_sleep(1);
  }
}

// A hand-over produced by every workgroup of the grid (workgroup w adds to sub-counter w % 8).
__device__ __forceinline__ void wait_grid(const BCtx& c, int li, int k) {
  wait_handover(c.s, c.ho(li, k), c.G / N_SUB, c.G % N_SUB);
}

// The h2 hand-over: from every workgroup, or with the 2-D down projection from
// the one workgroup per row group n that sums its K quarters (sub-counter n % 8).
__device__ __forceinline__ void wait_h2(const BCtx& c, int li) {
  if (c.d2) wait_handover(c.s, c.ho(li, HO_H2), c.dng / N_SUB, c.dng % N_SUB);
  else wait_grid(c, li, HO_H2);
}

// ---------------------------------------------------------------------------
// Operand movement
// ---------------------------------------------------------------------------

// The B-operand pieces of one weight unit of N k-steps: lane l holds row
// row + l%16 (rows >= row_end read zero without a memory access) at columns
// k0 + s*32 + (l/16)*8 .. +7 for k-step s (k0 a multiple of 32).
// Row-major matrices: each load reads 64 bytes from each of 16 rows.
// Tiled matrices (1 KiB block per 16 rows x 32 columns, lane order inside):
// each load reads one block, contiguous (streams ~20% faster).
template <int N>
__device__ __forceinline__ void load_w(rsrc_t r, bool tiled, int row, int row_end, uint32_t row_bytes, int k0,
                                       u32x4 (&wv)[N]) {
  const int lane = lane_id();
  const int n = row + (lane & 15);
  uint32_t o, step;
  if (tiled) {
    const uint32_t kb = row_bytes / 64u;   // k-steps (blocks) per 16-row tile
    o = (((uint32_t)n >> 4) * kb + ((uint32_t)k0 >> 5)) * 1024u + (uint32_t)(lane >> 4) * 256u + (uint32_t)(n & 15) * 16u;
    step = 1024u;
  } else {
    o = (uint32_t)n * row_bytes + (uint32_t)(k0 + (lane >> 4) * 8) * 2u;
    step = 64u;
  }
  if (n >= row_end) o = OOB;
#pragma unroll
  for (int s = 0; s < N; ++s) wv[s] = ld_stream(r, o + (uint32_t)s * step);
}

// att and act are exchanged in MFMA A-tile order (a_tile_off: 1 KiB per 16
// tokens x 32 columns, the 16 bytes each lane feeds to the MFMA contiguous),
// so the A loads of the O and down projections read whole 128-byte runs
// instead of 64 bytes from each token row.
// The A-operand pieces of N k-steps from such a matrix with kb = columns / 32
// (lane l: token mt*16 + l%16, columns k0 + s*32 + (l/16)*8 .. +7 for k-step s).
template <int MT, int N>
__device__ __forceinline__ void load_a_tiled(rsrc_t r, int B, int kb, int k0, u32x4 (&a)[MT * N]) {
  const int lane = lane_id();
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + (lane & 15);
    const uint32_t o = m < B ? ((uint32_t)(mt * kb + (k0 >> 5)) * 1024u + (uint32_t)lane * 16u) : OOB;
#pragma unroll
    for (int s = 0; s < N; ++s) a[mt * N + s] = ld16(r, o + (uint32_t)s * 1024u);
  }
}

// Stage the [B][2048] bf16 input of a phase into LDS with buffer loads to LDS
// (rows >= B zero), then RMS-normalise every row in place, keeping the raw
// columns [r0, r1) in L.res:
//   xn = bf16(x * rsqrt(mean(x^2) + eps))               (gamma folded into the weights)
//   xn = bf16(g * bf16(x * rsqrt(mean(x^2) + eps)))     (final norm, gamma g)
// src: an exchange buffer or hidden_in (row b at b*4096 bytes), or the
// embedding table (gather: row of token L.tok[b]).
// The staging copies of stage_norm (issued by stage_issue), then the
// normalisation (stage_finish). `after` runs between them: loads issued there
// (a fixed count, AFTER of them) are not waited for, since vector loads
// complete in order.
template <int MT>
__device__ __forceinline__ void stage_issue(const BCtx& c, rsrc_t src, bool gather, BLds<MT>& L,
                                            u32x4* hi_spare = nullptr) {
  const int wave = wave_id(), lane = lane_id();
  // 1 KiB quarters of rows: wave w copies quarters w, w+4, ... (16*MT each);
  // rows >= B read zero, into hi_spare instead when it is given
#pragma unroll
  for (int j = 0; j < 16 * MT; ++j) {
    const int qi = j * NWAVE + wave, m = qi >> 2, qq = qi & 3;
    const uint32_t row = gather ? (uint32_t)L.tok[m < BATCH_MAX ? m : 0] : (uint32_t)m;
    const uint32_t off = m < c.B ? row * (uint32_t)(H * 2) + (uint32_t)(qq * 1024 + lane * 16) : OOB;
    void* dst = hi_spare && m >= c.B ? (void*)hi_spare : (void*)&L.xn[m][qq * 512];
    __builtin_amdgcn_raw_ptr_buffer_load_lds(src, (lds_ptr_t)dst, 16, off, 0, 0, 0);
  }
  // no memory access may move above the copies: stage_finish counts on them
  // being the oldest loads in flight
  asm volatile("" ::: "memory");
}
template <int AFTER>
__device__ __forceinline__ void wait_vm_after() {
  static_assert(AFTER >= 0 && AFTER < 64, "vmcnt range");
  // vmcnt(AFTER): bits 3:0 and 15:14; expcnt and lgkmcnt at their maxima (no wait)
  __builtin_amdgcn_s_waitcnt((AFTER & 15) | ((AFTER >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}
template <int MT, int AFTER = 0>
__device__ __forceinline__ void stage_finish(const BCtx& c, const uint16_t* gamma, int r0, int r1, BLds<MT>& L);
template <int MT>
__device__ __forceinline__ void stage_norm(const BCtx& c, rsrc_t src, bool gather, const uint16_t* gamma, int r0,
                                           int r1, BLds<MT>& L) {
  stage_issue<MT>(c, src, gather, L);
  stage_finish<MT, 0>(c, gamma, r0, r1, L);
}
// RMS normalisation of the staged rows in place, TPR threads per token row
// (16, 32 or 64: the batch's rows spread over all 256 threads), chunk q + TPR*i
// (i < 256/TPR) of 8 elements each for thread q of its row; rows >= B (zeros
// from the staging) are skipped. The lanes of a row first copy its raw columns
// [r0, r1) to L.res (a wave's LDS accesses complete in order, so before any lane
// overwrites them), then read their chunks into registers at once, sum the
// squares with v_dot2 into two accumulators and write the normalised chunks
// back from the same registers: one LDS read and one write per chunk, no branch
// in the loop.
template <int MT, int TPR, bool GAMMA>
__device__ __forceinline__ void norm_rows(const BCtx& c, const uint16_t* gamma, int r0, int r1, BLds<MT>& L) {
  constexpr int NCH = (H / 8) / TPR;
  const int q = tid() & (TPR - 1);
  for (int m = tid() / TPR; m < c.B; m += NT / TPR) {
    uint16_t* row = &L.xn[m][0];
    for (int col = r0 + q; col < r1; col += TPR) L.res[m][col - r0] = row[col];
    u32x4 x[NCH], gvs[GAMMA ? NCH : 1];
#pragma unroll
    for (int i = 0; i < NCH; ++i) x[i] = *reinterpret_cast<const u32x4*>(&row[(q + TPR * i) * 8]);
    if (GAMMA) {   // every chunk's gamma issued at once (one memory round trip for the row)
#pragma unroll
      for (int i = 0; i < NCH; ++i) gvs[i] = *reinterpret_cast<const u32x4*>(gamma + (q + TPR * i) * 8);
    }
    float ssa = 0.f, ssb = 0.f;
#pragma unroll
    for (int i = 0; i < NCH; i += 2) {
      ssa = dot8(x[i], x[i], ssa);
      ssb = dot8(x[i + 1], x[i + 1], ssb);
    }
    float ss = ssa + ssb;
    ss = sum_lanes8(ss);
    ss += dpp<DPP_ROR8>(ss);          // the 16 lanes of a DPP row
    if (TPR >= 32) ss = add_xor16(ss);
    if (TPR >= 64) ss = add_xor32(ss);
    const float inv = rsqrtf(ss * (1.0f / H) + EPS);
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int col = (q + TPR * i) * 8;
      uint32_t e[4] = {x[i].x, x[i].y, x[i].z, x[i].w};
      u32x4 gv = {0u, 0u, 0u, 0u};
      if (GAMMA) gv = gvs[i];
      const uint32_t g[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t n = cvt_bf2(bf_lo(e[k]) * inv, bf_hi(e[k]) * inv);
        e[k] = GAMMA ? cvt_bf2(bf_lo(g[k]) * bf_lo(n), bf_hi(g[k]) * bf_hi(n)) : n;
      }
      *reinterpret_cast<u32x4*>(&row[col]) = u32x4{e[0], e[1], e[2], e[3]};
    }
  }
}
template <int MT, int AFTER>
__device__ __forceinline__ void stage_finish(const BCtx& c, const uint16_t* gamma, int r0, int r1, BLds<MT>& L) {
  wait_vm_after<AFTER>();
  lds_sync();
  if (gamma) {   // the final norm (once per step)
    if (c.B <= NT / 64) norm_rows<MT, 64, true>(c, gamma, r0, r1, L);
    else if (c.B <= NT / 32) norm_rows<MT, 32, true>(c, gamma, r0, r1, L);
    else norm_rows<MT, 16, true>(c, gamma, r0, r1, L);
  } else {
    if (c.B <= NT / 64) norm_rows<MT, 64, false>(c, gamma, r0, r1, L);
    else if (c.B <= NT / 32) norm_rows<MT, 32, false>(c, gamma, r0, r1, L);
    else norm_rows<MT, 16, false>(c, gamma, r0, r1, L);
  }
  lds_sync();
}

// The QKV input staged (the copies before the AFTER last loads have landed),
// raw: the raw columns [r0, r1) copied to L.res as stage_finish does; the
// normalisation is qkv_norm_a's.
template <int MT, int AFTER>
__device__ __forceinline__ void stage_wait_raw(const BCtx& c, int r0, int r1, BLds<MT>& L) {
  wait_vm_after<AFTER>();
  lds_sync();
  const int w = r1 - r0;
  for (int i = tid(); i < c.B * w; i += NT) L.res[i / w][i % w] = L.xn[i / w][r0 + i % w];
}
// The A operands of the QKV split-K MFMA (wave w: the K quarter [512w, 512w+512)
// of every row, in mma_lds's lane layout: a[mt*KS + s]) read from the raw
// staged rows and RMS-normalised in registers: x_n = bf16(x * rsqrt(mean(x^2) +
// eps)), the value norm_rows writes (gamma folded into the weights). Each
// wave sums the squares of its quarter from the operands it already holds (the
// 4 lanes of a row cover its 4 column chunks), the 4 waves' row sums meet in
// L.ssq (one barrier, summed in wave order), and each element is scaled by
// the lane that feeds it to the MFMA: no LDS write-back, no second barrier.
template <int MT>
__device__ __forceinline__ void qkv_norm_a(BLds<MT>& L, u32x4 (&a)[MT * KS]) {
  const int wave = wave_id(), lane = lane_id(), k0 = wave * KQ;
  float sa[MT], sb[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) sa[mt] = sb[mt] = 0.f;
#pragma unroll
  for (int s = 0; s < KS; ++s)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      a[mt * KS + s] = *reinterpret_cast<const u32x4*>(&L.xn[mt * 16 + (lane & 15)][k0 + s * 32 + (lane >> 4) * 8]);
      if (s & 1) sb[mt] = dot8(a[mt * KS + s], a[mt * KS + s], sb[mt]);
      else sa[mt] = dot8(a[mt * KS + s], a[mt * KS + s], sa[mt]);
    }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const float ss = add_xor32(add_xor16(sa[mt] + sb[mt]));   // row mt*16 + lane%16, this wave's quarter
    if (lane < 16) L.ssq[wave][mt * 16 + lane] = ss;
  }
  lds_sync();
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int r = mt * 16 + (lane & 15);
    const float ss = ((L.ssq[0][r] + L.ssq[1][r]) + L.ssq[2][r]) + L.ssq[3][r];
    const float inv = rsqrtf(ss * (1.0f / H) + EPS);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const u32x4 x = a[mt * KS + s];
      const uint32_t e[4] = {x.x, x.y, x.z, x.w};
      uint32_t o[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) o[k] = cvt_bf2(bf_lo(e[k]) * inv, bf_hi(e[k]) * inv);
      a[mt * KS + s] = u32x4{o[0], o[1], o[2], o[3]};
    }
  }
}

// One unit of MFMAs: KS k-steps from column k0, A from the staged LDS matrix.
template <int MT>
__device__ __forceinline__ void mma_lds(const BLds<MT>& L, int k0, const u32x4 (&wv)[KS], f32x4 (&acc)[MT]) {
  const int lane = lane_id();
#pragma unroll
  for (int s = 0; s < KS; ++s)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const u32x4 a = *reinterpret_cast<const u32x4*>(&L.xn[mt * 16 + (lane & 15)][k0 + s * 32 + (lane >> 4) * 8]);
      acc[mt] = mfma16(a, wv[s], acc[mt]);
    }
}
// One unit of MFMAs with the A operand in registers (a[mt*N + s]).
template <int MT, int N>
__device__ __forceinline__ void mma_reg(const u32x4 (&a)[MT * N], const u32x4 (&wv)[N], f32x4 (&acc)[MT]) {
#pragma unroll
  for (int s = 0; s < N; ++s)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = mfma16(a[mt * N + s], wv[s], acc[mt]);
}

// Paired operand loads, for a workgroup with at most 8 weight rows R0.. and at
// most 8 tokens (one token tile): rows (tokens) fill only half of the MFMA's 16
// operand lanes, so a plain load reads 512 useful bytes per KiB of lanes. Here
// lane l reads weight row R0 + l%8 (token l%8) of k-step 2j + (l/8)%2, columns
// (l/16)*8 .. +7: one load carries the operands of two k-steps, and mfma_pair
// moves the second into lanes l%16 < 8 with a DPP row rotation by 8. The other
// lanes' products land in output rows / columns that are discarded.
// Lane offset of k-step 0 in a weight matrix of row_bytes per row (rows >= R1
// out of range); k-step ks adds ks * pair_wstep.
__device__ __forceinline__ uint32_t pair_w_off(bool tiled, int R0, int R1, uint32_t row_bytes) {
  const int lane = lane_id(), n = R0 + (lane & 7), kh = (lane >> 3) & 1, ch = lane >> 4;
  uint32_t o;
  if (tiled) {
    const uint32_t kb = row_bytes / 64u;   // k-steps (1 KiB blocks) per 16-row tile
    o = (((uint32_t)n >> 4) * kb + (uint32_t)kh) * 1024u + (uint32_t)ch * 256u + (uint32_t)(n & 15) * 16u;
  } else {
    o = (uint32_t)n * row_bytes + (uint32_t)(kh * 32 + ch * 8) * 2u;
  }
  return n < R1 ? o : OOB;
}
__device__ __forceinline__ uint32_t pair_wstep(bool tiled) { return tiled ? 1024u : 64u; }
// Lane offset of k-step 0 in a matrix in A-tile order (a_tile_off; tokens >= B
// out of range); k-step ks adds ks * 1024.
__device__ __forceinline__ uint32_t pair_a_off(int B) {
  const int lane = lane_id(), t = lane & 7, kh = (lane >> 3) & 1, ch = lane >> 4;
  return t < B ? (uint32_t)kh * 1024u + (uint32_t)(ch * 16 + t) * 16u : OOB;
}
__device__ __forceinline__ f32x4 mfma_pair(u32x4 a0, u32x4 b0, f32x4 acc) {
  const u32x4 a1 = {dpp_u32<DPP_ROR8>(a0.x), dpp_u32<DPP_ROR8>(a0.y), dpp_u32<DPP_ROR8>(a0.z),
                    dpp_u32<DPP_ROR8>(a0.w)};
  const u32x4 b1 = {dpp_u32<DPP_ROR8>(b0.x), dpp_u32<DPP_ROR8>(b0.y), dpp_u32<DPP_ROR8>(b0.z),
                    dpp_u32<DPP_ROR8>(b0.w)};
  acc = mfma16(a0, b0, acc);
  return mfma16(a1, b1, acc);
}

// Sum of the 4 waves' partial tiles of token tile mt (fixed order, wave 0
// first), for any wave. The caller synchronises before L.red is reused.
template <int MT>
__device__ __forceinline__ f32x4 reduce_tile(const f32x4 (&acc)[MT], BLds<MT>& L, int mt) {
  const int wave = wave_id(), lane = lane_id();
#pragma unroll
  for (int m = 0; m < MT; ++m) L.red[wave][m][lane] = acc[m];
  lds_sync();
  f32x4 d = L.red[0][mt][lane];
#pragma unroll
  for (int w = 1; w < NWAVE; ++w) d += L.red[w][mt][lane];
  return d;
}

// A reduced tile's outputs: f(m, v) gets the token m (in the batch) and the
// summed value (reduce_tile's) of each of a lane's 4 output rows (lane/16)*4 + i.
// SPREAD: every wave finishes a share (wave w: token tile w % MT, 4*MT/4 of the
// rows); otherwise wave w < MT finishes all of token tile w (measured better
// with two tiles, where the share is two rows).
template <int MT, bool SPREAD, class F>
__device__ __forceinline__ void tile_out(const f32x4 (&acc)[MT], BLds<MT>& L, F&& f) {
  const int wave = wave_id(), lane = lane_id();
  if (SPREAD) {
    constexpr int IPW = 4 * MT / NWAVE;
    static_assert(IPW >= 1 && 4 * MT % NWAVE == 0, "tile output split");
    const int mtw = wave % MT, i0 = (wave / MT) * IPW;
    const f32x4 d = reduce_tile<MT>(acc, L, mtw);
#pragma unroll
    for (int ii = 0; ii < IPW; ++ii) {
      const int i = i0 + ii;
      f(mtw * 16 + (lane >> 4) * 4 + i, i == 0 ? d[0] : i == 1 ? d[1] : i == 2 ? d[2] : d[3]);
    }
  } else {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) L.red[wave][mt][lane] = acc[mt];
    lds_sync();
    if (wave < MT) {
      f32x4 d = L.red[0][wave][lane];
#pragma unroll
      for (int w = 1; w < NWAVE; ++w) d += L.red[w][wave][lane];
#pragma unroll
      for (int i = 0; i < 4; ++i) f(wave * 16 + (lane >> 4) * 4 + i, d[i]);
    }
  }
}

// ---------------------------------------------------------------------------
// Phases
// ---------------------------------------------------------------------------

// The work that depends on the positions only: each token's RoPE row (loaded
// into registers first, written to LDS last, so the loads overlap the plan) and
// the attention work plan (wave 0). With one MFMA tile it runs while the first
// layer's weight ring and input staging are in flight.
template <int MT>
__device__ __forceinline__ void plan_and_rope(BCtx& c, BLds<MT>& L) {
  const BParams& p = *c.p;
  const int t = tid();
  constexpr int RPT = (16 * MT * HD + NT - 1) / NT;   // RoPE words per thread at most
  uint32_t rv[RPT];
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    const int i = t + k * NT, m = i / HD;
    rv[k] = 0u;
    if (i < c.B * HD) {
      const int ps = L.pos[m];
      if (ps >= 0 && ps < p.rope_rows) rv[k] = reinterpret_cast<const uint32_t*>(p.rope + (size_t)ps * (2 * HD))[i % HD];
    }
  }
  if (wave_id() == 0) {
    // Attention work plan. The KV rows of every (sequence, kv head) form a
    // segment of 128-row groups (an attention item's unit of work: a partial
    // group costs a full one). Each segment is cut into p_b pieces of whole
    // groups, as equal as possible; a piece is one item. Every item beyond the
    // first on a workgroup costs a few us of fixed work (q hand-over, partial
    // publication, merge), so the plan is the smallest piece size m (in
    // groups, found by bisection) whose items fit one round of the grid: p_b = ceil(groups_b / m), at most 16 splits per segment. Items are
    // listed (sequence, kv head, piece). Lane b of wave 0 plans sequence b, in
    // 32-bit arithmetic (s_max <= 2^20 and batch <= 32 keep every count below
    // 2^25).
    const int lane = lane_id();
    const bool on = lane < c.B;
    const uint32_t n = on ? (uint32_t)L.pos[lane] + 1u : 0u;
    const uint32_t ng = (n + ATT_GROUP - 1u) / ATT_GROUP;      // 128-row groups per kv head
    const uint32_t max_ng = wave_max_u32(ng);
    const uint32_t slots = (uint32_t)c.G;
    auto pieces = [&](uint32_t m) { return on ? (ng + m - 1u) / m : 0u; };
    uint32_t lo = (max_ng + BATT_MAX_SPLIT - 1u) / BATT_MAX_SPLIT, hi = max_ng;   // <= 16 splits per segment
    if (lo < 1u) lo = 1u;
    if (hi < lo) hi = lo;
    while (lo < hi) {
      const uint32_t mid = (lo + hi) / 2u;
      if (wave_sum_u32((uint32_t)NKV * pieces(mid)) <= slots) hi = mid;
      else lo = mid + 1u;
    }
    const uint32_t pb = pieces(hi);
    const uint32_t items = (uint32_t)NKV * pb;
    const uint32_t incl = wave_incl_scan_u32(items);
    if (on) {
      L.ns[lane] = (int)pb;
      L.ng[lane] = (int)ng;
      L.cum[lane + 1] = (int)incl;
    }
    if (lane == 0) L.cum[0] = 0;
  }
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    const int i = t + k * NT;
    if (i < c.B * HD) reinterpret_cast<uint32_t*>(L.rope[i / HD])[i % HD] = rv[k];
  }
}

// QKV: RMSNorm of the layer input, [Wq;Wk;Wv] GEMM (split-K over the waves),
// RoPE at each sequence's position; q and the fresh K/V rows to the exchange
// buffer, K/V also into the caches at row pos[b] of sequence b.
// The first tile's weight unit of the QKV phase of run-layer li (issued by
// the caller: for the first layer at kernel start, before anything waits).
template <int MT>
__device__ __forceinline__ void qkv_first_unit(const BCtx& c, int li, u32x4 (&wv)[KS]) {
  const BParams& p = *c.p;
  int P0, P1;
  share(QKV_PAIRS, c.G, c.w, P0, P1);
  const int row0 = 2 * P0, row_end = 2 * P1;
  const rsrc_t rw = make_rsrc(p.w_qkv + (size_t)(p.first_layer + li) * QKV_ROWS * H, QKV_LAYER_BYTES);
  load_w<KS>(rw, p.tiled, row_end > row0 ? row0 : row_end, row_end, H * 2, wave_id() * KQ, wv);
}
// FIRST: the first layer (its weight unit already issued, its input final
// data); the others issue their unit here and wait for the previous layer's h2.
template <int MT, bool FIRST>
__device__ __forceinline__ void phase_qkv(BCtx& c, int li, BLds<MT>& L, u32x4 (&wv)[KS]) {
  const BParams& p = *c.p;
  const int l = p.first_layer + li, wave = wave_id(), lane = lane_id();
  int P0, P1, R0, R1;
  share(QKV_PAIRS, c.G, c.w, P0, P1);
  share(H, c.G, c.w, R0, R1);
  const int row0 = 2 * P0, row_end = 2 * P1, ntile = (row_end - row0 + 15) / 16;
  const rsrc_t rw = make_rsrc(p.w_qkv + (size_t)l * QKV_ROWS * H, QKV_LAYER_BYTES);
  if (!FIRST) qkv_first_unit<MT>(c, li, wv);
  trace_mark(c.s, 2 * xk(li, 1) - 1);
  if (!FIRST) {
    wait_h2(c, li - 1);
    stage_issue<MT>(c, make_rsrc(c.xb(li - 1, p.lay.h2), (size_t)c.B * H * 2), false, L);
    stage_wait_raw<MT, 0>(c, R0, R1, L);
  } else {   // the first layer: its input is final data; the plan runs while it lands
    if (p.hidden_in) stage_issue<MT>(c, make_rsrc(p.hidden_in, (size_t)c.B * H * 2), false, L);
    else stage_issue<MT>(c, make_rsrc(p.embed, EMBED_BYTES), true, L);
    if (MT == 1) plan_and_rope<MT>(c, L);   // (two tiles: in the prologue; inlined here it spills)
    stage_wait_raw<MT, 0>(c, R0, R1, L);
  }
  // each wave normalises the K quarter it multiplies, in its A-operand registers
  u32x4 an[MT * KS];
  qkv_norm_a<MT>(L, an);
  trace_mark(c.s, 2 * xk(li, 1));
  uint16_t* xq = c.sx(li, p.lay.sq_qkv);
  for (int tt = 0; tt < ntile; ++tt) {
    f32x4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    mma_reg<MT, KS>(an, wv, acc);
    if (tt + 1 < ntile) load_w<KS>(rw, p.tiled, row0 + 16 * (tt + 1), row_end, H * 2, wave * KQ, wv);
    // every wave finishes a share of the outputs: token tile wave % MT, and
    // IPW of the 4 output rows of each lane (rows (lane/16)*4 + i of the tile)
    constexpr int IPW = 4 * MT / NWAVE;
    static_assert(IPW >= 1 && 4 * MT % NWAVE == 0, "QKV epilogue split");
    const int mtw = wave % MT, i0 = (wave / MT) * IPW;
    const f32x4 d = reduce_tile<MT>(acc, L, mtw);
    {
      const int row = row0 + tt * 16 + (lane & 15);
      const bool rv = row < row_end;
      const int pr = row >> 1, dd = pr & 31, hi = row & 1;
#pragma unroll
      for (int ii = 0; ii < IPW; ++ii) {
        const int i = i0 + ii;
        const float di = i == 0 ? d[0] : i == 1 ? d[1] : i == 2 ? d[2] : d[3];
        const float mine = rbf(di);
        const float other = dpp<DPP_XOR1>(mine);   // the pair partner (row ^ 1)
        const int m = mtw * 16 + (lane >> 4) * 4 + i;
        if (!rv || m >= c.B) continue;
        const float a = hi ? other : mine, b = hi ? mine : other;   // elements d, d+32
        const int ps = L.pos[m];
        uint32_t outv;
        if (pr < Q_PAIRS + K_PAIRS) {
          const u32x4 o = rope_pair(a, b, L.rope[m], dd);
          outv = hi ? o.y : o.x;
        } else {
          outv = f2bf(mine);
        }
        int col;
        if (pr < Q_PAIRS) {
          col = (pr >> 5) * HD + dd + 32 * hi;
        } else {
          const bool is_k = pr < Q_PAIRS + K_PAIRS;
          const int kh = (pr - Q_PAIRS - (is_k ? 0 : K_PAIRS)) >> 5;
          col = NQ * HD + (is_k ? 0 : NKV * HD) + kh * HD + dd + 32 * hi;
          // device scope: in a prefill step the other tokens' attention reads this row
          uint16_t* crow =
              (is_k ? p.kc[li] : p.vc[li]) + ((size_t)(c.cache_seq(m) * NKV + kh) * p.s_max + ps) * HD + dd + 32 * hi;
          st_dev(crow, outv);
        }
        st_dev(xq + (size_t)m * QKV_ROWS + col, outv);
      }
    }
    lds_sync();   // L.red reuse
  }
  // decode steps: the attention items poll q and the fresh K/V rows; a prefill
  // step's attention also reads cache rows other workgroups write in this
  // launch, so it waits for every workgroup's stores (an arrival counter)
  if (c.prefill) arrive(c.ho(li, HO_QKV), c.w % N_SUB);
  trace_done(c.s, li, 0);
}

// Attention: the workgroup's items (sequence, kv head, split); the last split
// of a (sequence, kv head) to arrive merges its partials.
template <int MT>
__device__ __forceinline__ void phase_attn(BCtx& c, int li, BLds<MT>& L) {
  const BParams& p = *c.p;
  const int lane = lane_id(), t = tid();
  const int nitems = L.cum[c.B];
  const rsrc_t rq = make_rsrc(c.sx(li, p.lay.sq_qkv), (size_t)c.B * QKV_ROWS * 2);
  bool waited = false;
  // Round k of the grid takes items [k*G, (k+1)*G) (one round unless the grid
  // is small): workgroup w takes item k*G + w in even rounds and
  // k*G + G-1-w in odd ones (zig-zag).
  for (int rbase = 0, k = 0; rbase < nitems; rbase += c.G, ++k) {
    const int it = rbase + ((k & 1) ? c.G - 1 - c.w : c.w);
    if (it >= nitems) continue;
    {
      // the item's sequence: the number of sequences whose items all come
      // before it (cum is non-decreasing; one LDS read per lane and a ballot)
      const int lane_b = lane < c.B ? L.cum[lane + 1] : 0x7fffffff;
      const int b = __popcll(__ballot(lane_b <= it));
      const int nsb = L.ns[b], rr = it - L.cum[b], h = rr / nsb, sp = rr % nsb;
      const int ngb = L.ng[b];
      const int ga = sp * ngb / nsb, gb = (sp + 1) * ngb / nsb;   // the piece's groups
      const int ps = L.pos[b];
      const int j0 = ga * ATT_GROUP, j1 = min(gb * ATT_GROUP, ps + 1);
      const bool fresh = ps >= j0 && ps < j1;
      // the item's cached rows do not depend on this step: its first BATT_DEPTH groups are issued
      // before the wait for q (in a prefill step rows of this step's tokens are among them: issued after it)
      const size_t head = (size_t)(c.cache_seq(b) * NKV + h) * p.s_max * HD;
      AttnRows ar;
      ar.init(p.kc[li] + head, p.vc[li] + head, p.s_max, j0, min(j1, ps));
      AttnGroupMx ring[BATT_DEPTH + 1];
      auto issue_ahead = [&]() {
#pragma unroll
        for (int g = 0; g < BATT_DEPTH; ++g) load_mx(ar, g, ring[g]);
      };
      if (!c.prefill) issue_ahead();
      if (wave_id() == 0) {
        if (!waited) trace_mark(c.s, 2 * xk(li, 2) - 1);
        if (!waited && c.prefill) wait_grid(c, li, HO_QKV);
        // q of heads 4h..4h+3 (512 B, lanes 0-31), the fresh K row (lanes 32-39) and V row (40-47)
        const uint32_t base = (uint32_t)b * (QKV_ROWS * 2);
        uint32_t off[1];
        off[0] = lane < 32 ? base + (uint32_t)(h * GQA * HD * 2 + lane * 16)
               : lane < 40 ? (fresh ? base + (uint32_t)((NQ * HD + h * HD) * 2 + (lane - 32) * 16) : OOB)
               : lane < 48 ? (fresh ? base + (uint32_t)((NQ * HD + NKV * HD + h * HD) * 2 + (lane - 40) * 16) : OOB)
                           : OOB;
        u32x4 v[1];
        poll_bf16<1>(c.s, rq, off, v);   // (complete at once after a prefill step's counter)
        if (!waited) trace_mark(c.s, 2 * xk(li, 2));
        if (lane < 48) *reinterpret_cast<u32x4*>(L.q + lane * 8) = v[0];
      }
      waited = true;
      lds_sync();
      if (c.prefill) issue_ahead();
      // the head's only split writes the final output, no partial (with two
      // MFMA tiles, where every head has one split at long contexts)
      const bool only = MT == 2 && nsb == 1;
      attn_item_mx<BATT_DEPTH>(ar, ring, L.q, fresh, c.part(li, b, h, sp), L.att,
                               only ? c.xb(li, p.lay.att) : nullptr, b, h * GQA * HD);
      if (only) {
        arrive(c.ho(li, HO_ATT), (b * NKV + h) % N_SUB);
        continue;
      }
      // publish the partial and count it in; the last arrival merges
      wait_mem();
      lds_sync();
      if (t == 0) {
        uint32_t* cp = c.acnt + ((size_t)li * p.max_batch + b) * NKV + h;
        const uint32_t prev = __hip_atomic_fetch_add(cp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        L.flag = prev == (uint32_t)(nsb - 1);
      }
      lds_sync();
      if (L.flag) {
        // (instantiated for the segment's split count: every slot up to MAXS is a load)
        float* ph = c.part(li, b, h, 0);
        uint16_t* att = c.xb(li, p.lay.att);
        if (nsb <= 4) attn_merge_head<false, 4, true>(c.s, ph, nsb, att, b, h * GQA * HD);
        else if (nsb <= 8) attn_merge_head<false, 8, true>(c.s, ph, nsb, att, b, h * GQA * HD);
        else attn_merge_head<false, BATT_MAX_SPLIT, true>(c.s, ph, nsb, att, b, h * GQA * HD);
        arrive(c.ho(li, HO_ATT), (b * NKV + h) % N_SUB);
      }
    }
  }
  if (waited) trace_done(c.s, li, 1);
}

// O projection (split-K, A = attention output read in MFMA layout) + residual -> h1.
template <int MT>
__device__ __forceinline__ void phase_o(BCtx& c, int li, BLds<MT>& L, GuCopy& guc) {
  const BParams& p = *c.p;
  const int l = p.first_layer + li, wave = wave_id(), lane = lane_id();
  int R0, R1;
  share(H, c.G, c.w, R0, R1);
  const int ntile = (R1 - R0 + 15) / 16;
  const rsrc_t rw = make_rsrc(p.w_o + (size_t)l * H * H, O_LAYER_BYTES);
  // at most 8 rows and 8 tokens: paired operand loads (pair_w_off), half the loads
  const bool pr = MT == 1 && c.dpair && c.B <= 8;
  const uint32_t wo = pair_w_off(p.tiled, R0, R1, H * 2), wstep = pair_wstep(p.tiled);
  const int ks0 = wave * (KQ / 32);
  u32x4 wv[KS];
  if (pr) {
#pragma unroll
    for (int j = 0; j < KS / 2; ++j) wv[j] = ld_stream(rw, wo + (uint32_t)(ks0 + 2 * j) * wstep);
  } else {
    load_w<KS>(rw, p.tiled, ntile > 0 ? R0 : R1, R1, H * 2, wave * KQ, wv);
  }
  trace_mark(c.s, 2 * xk(li, 3) - 1);
  // every (sequence, kv head) merge adds to sub-counter (b*8 + h) % N_SUB
  if constexpr (BLds<MT>::GW > 1)
    wait_handover_copy(c.s, c.ho(li, HO_ATT), c.B * NKV / N_SUB, c.B * NKV % N_SUB, guc, BGU_CH_O,
                       &L.gw[wave * KS * 64], BGU_SKIP_O);
  else
    wait_handover(c.s, c.ho(li, HO_ATT), c.B * NKV / N_SUB, c.B * NKV % N_SUB);
  trace_mark(c.s, 2 * xk(li, 3));
  const rsrc_t ratt = make_rsrc(c.xb(li, p.lay.att), (size_t)((c.B + 15) / 16 * 16) * H * 2);
  uint16_t* h1 = c.xb(li, p.lay.h1);
  if (pr) {
    const uint32_t ao = pair_a_off(c.B);
    u32x4 a[KS / 2];
#pragma unroll
    for (int j = 0; j < KS / 2; ++j) a[j] = ld16(ratt, ao + (uint32_t)(ks0 + 2 * j) * 1024u);
    f32x4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KS / 2; ++j) acc[0] = mfma_pair(a[j], wv[j], acc[0]);
    const int row = R0 + (lane & 15);
    tile_out<MT, true>(acc, L, [&](int m, float v) {
      if (row < R1 && m < c.B) st_dev(h1 + (size_t)m * H + row, f2bf(bf2f(L.res[m][row - R0]) + rbf(v)));
    });
    lds_sync();
    arrive(c.ho(li, HO_H1), c.w % N_SUB);
    trace_done(c.s, li, 2);
    return;
  }
  u32x4 a[MT * KS];
  load_a_tiled<MT, KS>(ratt, c.B, H / 32, wave * KQ, a);
  for (int tt = 0; tt < ntile; ++tt) {
    f32x4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    mma_reg<MT, KS>(a, wv, acc);
    if (tt + 1 < ntile) load_w<KS>(rw, p.tiled, R0 + 16 * (tt + 1), R1, H * 2, wave * KQ, wv);
    const int row = R0 + tt * 16 + (lane & 15);
    tile_out<MT, false>(acc, L, [&](int m, float v) {
      if (row < R1 && m < c.B) st_dev(h1 + (size_t)m * H + row, f2bf(bf2f(L.res[m][row - R0]) + rbf(v)));
    });
    lds_sync();
  }
  arrive(c.ho(li, HO_H1), c.w % N_SUB);
  trace_done(c.s, li, 2);
}

// The LDS copy of the last weight unit of the wave's gate/up tile of run-layer
// li (one token tile and exactly one tile per wave; otherwise no copy). It is
// started in the O phase's wait for the attention output and finished in the
// gate/up phase's h1 wait.
template <int MT>
__device__ __forceinline__ void gu_copy_init(const BCtx& c, int li, BLds<MT>& L, GuCopy& gc) {
  const BParams& p = *c.p;
  int U0, U1;
  share(INTER, c.G, c.w, U0, U1);
  const int row0 = 2 * U0, row_end = 2 * U1, ntile = (row_end - row0 + 15) / 16, wave = wave_id();
  const int my_tiles = ntile > wave ? (ntile - wave + NWAVE - 1) / NWAVE : 0;
  const rsrc_t rw = make_rsrc(p.w_gu + (size_t)(p.first_layer + li) * 2 * INTER * H, GU_LAYER_BYTES);
  constexpr bool GL = BLds<MT>::GW > 1;
  gc.u3.init(rw, p.tiled, row0 + 16 * wave, row_end, H * 2, (H / (KS * 32) - 1) * KS * 32, GL && my_tiles == 1);
  gc.half = GL && c.B <= 8 && ntile == NWAVE;
  gc.u2.init(rw, p.tiled, row0 + 16 * wave, row_end, H * 2, 2 * KS * 32, gc.half);
  gc.d3 = &L.gw[GL ? wave * KS * 64 : 0];
  gc.d2 = reinterpret_cast<u32x4*>(&L.xn[MT == 1 ? 8 : 0][0]) + wave * (KS / 2) * 64;
}

// RMSNorm(h1) -> gate/up GEMM (whole tiles per wave) -> silu(gate) * up -> act.
template <int MT>
__device__ __forceinline__ void phase_gu(BCtx& c, int li, BLds<MT>& L, GuCopy& gc) {
  const BParams& p = *c.p;
  const int l = p.first_layer + li, wave = wave_id(), lane = lane_id();
  int U0, U1, R0, R1;
  share(INTER, c.G, c.w, U0, U1);
  share(H, c.G, c.w, R0, R1);
  const int row0 = 2 * U0, row_end = 2 * U1, ntile = (row_end - row0 + 15) / 16;
  constexpr int UPT = H / (KS * 32);   // 4 units per tile
  const int my_tiles = ntile > wave ? (ntile - wave + NWAVE - 1) / NWAVE : 0;
  const int nunits = my_tiles * UPT;
  const rsrc_t rw = make_rsrc(p.w_gu + (size_t)l * 2 * INTER * H, GU_LAYER_BYTES);
  auto issue = [&](int u, u32x4(&wv)[KS]) {
    load_w<KS>(rw, p.tiled, u < nunits ? row0 + 16 * (wave + NWAVE * (u / UPT)) : row_end, row_end, H * 2,
               (u % UPT) * KS * 32, wv);
  };
  u32x4 wa[KS], wb[KS];
  // With one token tile, a wave with one weight tile takes that tile's last
  // unit from the LDS copy gc.u3 (gu_copy_init), made during the waits for the
  // attention output and h1 (HBM is mostly idle then); the copies those waits
  // leave are issued behind the staging.
  constexpr bool GL = BLds<MT>::GW > 1;
  static_assert(UPT == 4, "gate/up unit schedule");
  const bool gl = GL && nunits == UPT;
  u32x4* gdst = gc.d3;
  u32x4* spare = &L.gspare[GL ? wave * 64 : 0];
  // with at most 8 tokens, the first half of unit 2 is in LDS too (gc.u2)
  const bool half = gl && gc.half;
  // one weight unit is issued before the h1 wait, the other right behind the
  // h1 staging copies, so the staging does not queue behind it
  issue(0, wa);
  trace_mark(c.s, 2 * xk(li, 4) - 1);
  if (GL) wait_handover_copy(c.s, c.ho(li, HO_H1), c.G / N_SUB, c.G % N_SUB, gc, BGU_CH, gdst);
  else wait_grid(c, li, HO_H1);
  stage_issue<MT>(c, make_rsrc(c.xb(li, p.lay.h1), (size_t)c.B * H * 2), false, L, gc.half ? spare : nullptr);
  issue(1, wb);
  if (GL) {
    gc.u3.issue_fixed<KS>(gdst, spare);
    gc.u2.issue_fixed<KS / 2>(gc.d2, spare);
  }
  // the raw columns kept for the down projection's residual: its rows
  const int D0 = c.d2 ? (c.w / DN_KQ) * c.drpg : R0, D1 = c.d2 ? D0 + c.drpg : R1;
  stage_finish<MT, KS + (GL ? KS + KS / 2 : 0)>(c, nullptr, D0, D1, L);
  trace_mark(c.s, 2 * xk(li, 4));
  uint16_t* act = c.xb(li, p.lay.act);
  f32x4 acc[MT];
  auto unit = [&](int u, u32x4(&wv)[KS], bool refill) {
    if (u % UPT == 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    mma_lds<MT>(L, (u % UPT) * KS * 32, wv, acc);
    if (refill) issue(u + 2, wv);
    if (u % UPT == UPT - 1) {
      const int row = row0 + 16 * (wave + NWAVE * (u / UPT)) + (lane & 15);
      const bool gate = (row & 1) == 0;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float mine = acc[mt][i];
          const float other = dpp<DPP_XOR1>(mine);   // up (row + 1) for a gate lane
          const int m = mt * 16 + (lane >> 4) * 4 + i;
          if (gate && row < row_end && m < c.B)
            st_dev(act + a_tile_off(m, row >> 1, INTER / 32), f2bf(mine / (1.0f + __expf(-mine)) * other));
        }
    }
  };
  if (half) {   // units 0, 1 and the second half of 2 from registers, the rest from LDS
    unit(0, wa, false);
    load_w<KS / 2>(rw, p.tiled, row0 + 16 * wave, row_end, H * 2, 2 * KS * 32 + (KS / 2) * 32,
                   *reinterpret_cast<u32x4(*)[KS / 2]>(&wa[KS / 2]));
    unit(1, wb, false);
    wait_mem();   // the copies were issued before these loads
#pragma unroll
    for (int s = 0; s < KS / 2; ++s) wa[s] = gc.d2[s * 64 + lane];
    unit(2, wa, false);
#pragma unroll
    for (int s = 0; s < KS; ++s) wa[s] = gdst[s * 64 + lane];
    unit(3, wa, false);
  } else if (gl) {   // units 0-2 from registers (unit 2 issued after unit 0), unit 3 from LDS
    unit(0, wa, true);
    unit(1, wb, false);
    unit(2, wa, false);
    wait_mem();   // the copies were issued before unit 2's loads
#pragma unroll
    for (int s = 0; s < KS; ++s) wa[s] = gdst[s * 64 + lane];
    unit(3, wa, false);
  } else {
    for (int u = 0; u < nunits; u += 2) {
      unit(u, wa, true);
      if (u + 1 < nunits) unit(u + 1, wb, true);
    }
  }
  arrive(c.ho(li, HO_ACT), c.w % N_SUB);
  trace_done(c.s, li, 3);
}

// Down projection (split-K over the waves, A = act read in MFMA layout) + residual -> h2.
template <int MT>
__device__ __forceinline__ void phase_down(BCtx& c, int li, BLds<MT>& L) {
  const BParams& p = *c.p;
  // (the thread index read opaquely in every translation unit, tid_opaque():
  // the one-tile kernel measured 0.8% faster with it in the down projections)
  const unsigned tix = tid_opaque();
  const int l = p.first_layer + li, wave = (int)(tix >> 6), lane = (int)(tix & 63u);
  const bool last = li == p.n_layers - 1;
  int R0, R1;
  share(H, c.G, c.w, R0, R1);
  const int ntile = (R1 - R0 + 15) / 16;
  constexpr int KW = INTER / NWAVE;       // 2048 columns per wave
  constexpr int UPT = KW / (DKS * 32);    // 8 units per tile
  const int nunits = ntile * UPT;
  const rsrc_t rw = make_rsrc(p.w_d + (size_t)l * H * INTER, D_LAYER_BYTES);
  const rsrc_t ra = make_rsrc(c.xb(li, p.lay.act), (size_t)((c.B + 15) / 16 * 16) * INTER * 2);
  struct Unit {
    u32x4 w[DKS];
    u32x4 a[MT * DKS];
  };
  auto issue_w = [&](int u, Unit& un) {
    load_w<DKS>(rw, p.tiled, u < nunits ? R0 + 16 * (u / UPT) : R1, R1, INTER * 2, wave * KW + (u % UPT) * DKS * 32, un.w);
  };
  auto issue_a = [&](int u, Unit& un) {
    load_a_tiled<MT, DKS>(ra, u < nunits ? c.B : 0, INTER / 32, wave * KW + (u % UPT) * DKS * 32, un.a);
  };
  Unit ua, ub;
  issue_w(0, ua);
  issue_w(1, ub);
  trace_mark(c.s, 2 * xk(li, 5) - 1);
  wait_grid(c, li, HO_ACT);
  trace_mark(c.s, 2 * xk(li, 5));
  issue_a(0, ua);
  issue_a(1, ub);
  uint16_t* h2 = c.xb(li, p.lay.h2);
  f32x4 acc[MT];
  auto unit = [&](int u, Unit& un) {
    if (u % UPT == 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    mma_reg<MT, DKS>(un.a, un.w, acc);
    issue_w(u + 2, un);
    issue_a(u + 2, un);
    if (u % UPT == UPT - 1) {
      const int row = R0 + (u / UPT) * 16 + (lane & 15);
      tile_out<MT, false>(acc, L, [&](int m, float v) {
        if (row < R1 && m < c.B) {
          const uint32_t hv = f2bf(bf2f(L.res[m][row - R0]) + rbf(v));
          st_dev(h2 + (size_t)m * H + row, hv);
          if (last && p.hidden_out) p.hidden_out[(size_t)m * H + row] = (uint16_t)hv;
        }
      });
      lds_sync();
    }
  };
  for (int u = 0; u < nunits; u += 2) {
    unit(u, ua);
    if (u + 1 < nunits) unit(u + 1, ub);
  }
  arrive(c.ho(li, HO_H2), c.w % N_SUB);
  trace_done(c.s, li, 4);
}

// The down projection of a workgroup with at most 8 rows (a 256-workgroup
// grid) at batches of at most 8, with paired operand loads (pair_w_off): same
// result as phase_down (same k order per wave), with twice the bytes in
// flight per register.
template <int MT>
__device__ __forceinline__ void phase_down_pair(BCtx& c, int li, BLds<MT>& L) {
  static_assert(MT == 1, "one token tile");
  const BParams& p = *c.p;
  // (the thread index read opaquely in every translation unit, tid_opaque():
  // the one-tile kernel measured 0.8% faster with it in the down projections)
  const unsigned tix = tid_opaque();
  const int l = p.first_layer + li, wave = (int)(tix >> 6), lane = (int)(tix & 63u);
  const bool last = li == p.n_layers - 1;
  int R0, R1;
  share(H, c.G, c.w, R0, R1);
  constexpr int KW = INTER / NWAVE;       // 2048 columns per wave
  constexpr int UPT = KW / (DKS * 32);    // 8 units (one tile)
  constexpr int NP = DKS / 2;             // k-step pairs per unit
  constexpr int NR = BDN_RING;
  static_assert(UPT % NR == 0 && BDN_PRE <= NR, "down ring");
  const rsrc_t rw = make_rsrc(p.w_d + (size_t)l * H * INTER, D_LAYER_BYTES);
  const rsrc_t ra = make_rsrc(c.xb(li, p.lay.act), (size_t)((c.B + 15) / 16 * 16) * INTER * 2);
  const uint32_t wo = pair_w_off(p.tiled, R0, R1, INTER * 2), wstep = pair_wstep(p.tiled);
  const uint32_t ao = pair_a_off(c.B);
  struct Unit {
    u32x4 w[NP];
    u32x4 a[NP];
  };
  auto issue_w = [&](int u, Unit& un) {
    const int ks0 = (wave * KW + u * DKS * 32) >> 5;   // first k-step of the unit
#pragma unroll
    for (int j = 0; j < NP; ++j)
      un.w[j] = ld_stream(rw, u < UPT ? wo + (uint32_t)(ks0 + 2 * j) * wstep : OOB);
  };
  auto issue_a = [&](int u, Unit& un) {
    const int ks0 = (wave * KW + u * DKS * 32) >> 5;
#pragma unroll
    for (int j = 0; j < NP; ++j) un.a[j] = ld16(ra, u < UPT ? ao + (uint32_t)(ks0 + 2 * j) * 1024u : OOB);
  };
  Unit ring[NR];
#pragma unroll
  for (int s = 0; s < BDN_PRE; ++s) issue_w(s, ring[s]);
  trace_mark(c.s, 2 * xk(li, 5) - 1);
  wait_grid(c, li, HO_ACT);
  trace_mark(c.s, 2 * xk(li, 5));
#pragma unroll
  for (int s = 0; s < NR; ++s) {
    if (s >= BDN_PRE) issue_w(s, ring[s]);
    issue_a(s, ring[s]);
  }
  f32x4 acc[1] = {f32x4{0.f, 0.f, 0.f, 0.f}};
  auto unit = [&](int u, Unit& un) {
#pragma unroll
    for (int j = 0; j < NP; ++j) acc[0] = mfma_pair(un.a[j], un.w[j], acc[0]);
    issue_w(u + NR, un);
    issue_a(u + NR, un);
  };
  for (int u = 0; u < UPT; u += NR) {
#pragma unroll
    for (int s = 0; s < NR; ++s) unit(u + s, ring[s]);
  }
  uint16_t* h2 = c.xb(li, p.lay.h2);
  const int row = R0 + (lane & 15);
  tile_out<MT, true>(acc, L, [&](int m, float v) {
    if (row < R1 && m < c.B) {
      const uint32_t hv = f2bf(bf2f(L.res[m][row - R0]) + rbf(v));
      st_dev(h2 + (size_t)m * H + row, hv);
      if (last && p.hidden_out) p.hidden_out[(size_t)m * H + row] = (uint16_t)hv;
    }
  });
  lds_sync();
  arrive(c.ho(li, HO_H2), c.w % N_SUB);
  trace_done(c.s, li, 4);
}

// Down projection as a 2-D split: workgroup w computes the rows of row group
// n = w / 4 over the K quarter kq = w % 4 (split over the 4 waves as above), so
// it reads a quarter of act instead of all of it and fills whole 16-row tiles.
// The four quarters' fp32 partials go to dpart; the workgroup that completes a
// row group last (an arrival counter) sums them in the fixed order kq = 0..3,
// adds the residual and publishes the rows of h2.
template <int MT>
__device__ __forceinline__ void phase_down2d(BCtx& c, int li, BLds<MT>& L) {
  const BParams& p = *c.p;
  const int l = p.first_layer + li, wave = wave_id(), lane = lane_id(), t = tid();
  const bool last = li == p.n_layers - 1;
  const int n = c.w / DN_KQ, kq = c.w % DN_KQ;
  const int R0 = n * c.drpg, R1 = R0 + c.drpg, ntile = c.drpg / 16;
  constexpr int KW = INTER / DN_KQ / NWAVE;   // 512 columns per wave
  constexpr int UPT = KW / (DKS * 32);         // 2 units per tile
  const int nunits = ntile * UPT;
  const int k0w = kq * (INTER / DN_KQ) + wave * KW;
  const rsrc_t rw = make_rsrc(p.w_d + (size_t)l * H * INTER, D_LAYER_BYTES);
  const rsrc_t ra = make_rsrc(c.xb(li, p.lay.act), (size_t)((c.B + 15) / 16 * 16) * INTER * 2);
  float* dp = c.dpart(li);
  struct Unit {
    u32x4 w[DKS];
    u32x4 a[MT * DKS];
  };
  auto issue_w = [&](int u, Unit& un) {
    load_w<DKS>(rw, p.tiled, u < nunits ? R0 + 16 * (u / UPT) : R1, R1, INTER * 2, k0w + (u % UPT) * DKS * 32, un.w);
  };
  auto issue_a = [&](int u, Unit& un) {
    load_a_tiled<MT, DKS>(ra, u < nunits ? c.B : 0, INTER / 32, k0w + (u % UPT) * DKS * 32, un.a);
  };
  Unit ua, ub;
  issue_w(0, ua);
  issue_w(1, ub);
  trace_mark(c.s, 2 * xk(li, 5) - 1);
  wait_grid(c, li, HO_ACT);
  trace_mark(c.s, 2 * xk(li, 5));
  issue_a(0, ua);
  issue_a(1, ub);
  f32x4 acc[MT];
  auto unit = [&](int u, Unit& un) {
    if (u % UPT == 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    mma_reg<MT, DKS>(un.a, un.w, acc);
    issue_w(u + 2, un);
    issue_a(u + 2, un);
    if (u % UPT == UPT - 1) {
      const int row = R0 + (u / UPT) * 16 + (lane & 15);
      tile_out<MT, false>(acc, L, [&](int m, float v) {
        if (m < c.B) st_dev(dp + ((size_t)kq * p.max_batch + m) * H + row, v);
      });
      lds_sync();
    }
  };
  for (int u = 0; u < nunits; u += 2) {
    unit(u, ua);
    if (u + 1 < nunits) unit(u + 1, ub);
  }
  // count this quarter in; the row group's last quarter sums the four
  wait_mem();
  lds_sync();
  if (t == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(c.dcnt + (size_t)li * DN_MAX + n, 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    L.flag = prev == (uint32_t)(DN_KQ - 1);
  }
  lds_sync();
  if (L.flag) {
    const rsrc_t rp = make_rsrc(dp, (size_t)DN_KQ * p.max_batch * H * 4);
    uint16_t* h2 = c.xb(li, p.lay.h2);
    // four consecutive rows per thread: the four quarters' 16-byte loads are in
    // flight together (drpg % 16 == 0, so a group never straddles two tokens)
    const int n4 = c.drpg / 4;
    for (int i = t; i < c.B * n4; i += NT) {
      const int m = i / n4, r = (i % n4) * 4, row = R0 + r;
      u32x4 v[DN_KQ];
#pragma unroll
      for (int q = 0; q < DN_KQ; ++q) v[q] = ld_dev16(rp, (uint32_t)((((size_t)q * p.max_batch + m) * H + row) * 4));
      uint32_t hv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float sum = 0.f;
#pragma unroll
        for (int q = 0; q < DN_KQ; ++q) sum += __uint_as_float(v[q][j]);
        hv[j] = f2bf(bf2f(L.res[m][r + j]) + rbf(sum));
      }
      const unsigned long long packed = (unsigned long long)(hv[0] | (hv[1] << 16)) |
                                        ((unsigned long long)(hv[2] | (hv[3] << 16)) << 32);
      __hip_atomic_store(reinterpret_cast<unsigned long long*>(h2 + (size_t)m * H + row), packed, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      if (last && p.hidden_out) {
#pragma unroll
        for (int j = 0; j < 4; ++j) p.hidden_out[(size_t)m * H + row + j] = (uint16_t)hv[j];
      }
    }
    arrive(c.ho(li, HO_H2), n % N_SUB);
  }
  trace_done(c.s, li, 4);
}

// Refill the other sentinel set (the next launch's) with the sentinel: nothing
// reads it before that launch, and the kernel boundary orders the two.
// Device-scope stores, so the next launch's polls find them in memory.
__device__ __forceinline__ void refill_sentinel_set(const BCtx& c, uint32_t epoch) {
  const BParams& p = *c.p;
  const rsrc_t r = make_rsrc(p.xch + p.lay.sent_base + (size_t)((epoch + 1u) & 1u) * p.lay.sset, p.lay.sset);
  int lo, hi;
  share((int)(p.lay.sset / 16), c.G, c.w, lo, hi);
  const u32x4 ones = {~0u, ~0u, ~0u, ~0u};
  for (int i = lo + (int)tid(); i < hi; i += NT)
    __builtin_amdgcn_raw_buffer_store_b128(ones, r, (int)((uint32_t)i * 16u), 0, AUX_SC1);
}

// Zero the other counter set (the next launch's) and refill its sentinel set:
// nothing in this launch uses either, so this runs where the stores delay no
// load (behind the lm_head stream, or after the last layer).
__device__ __forceinline__ void prepare_next_launch(const BCtx& c, uint32_t epoch) {
  refill_sentinel_set(c, epoch);
  int lo, hi;
  share(c.cnt_words, c.G, c.w, lo, hi);
  for (int i = lo + (int)tid(); i < hi; i += NT)
    __hip_atomic_store(c.cnt_other + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Maximum of a 64-bit value over each 16-lane DPP row, in every lane of the
// row: quad swaps, then rotations by 4 and 8 within the row (both halves moved
// by the same DPP control; no LDS round trip as a lane shuffle would take).
template <int CTRL>
__device__ __forceinline__ unsigned long long dpp_u64(unsigned long long v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, 0xf, 0xf, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, 0xf, 0xf, false);
  return ((unsigned long long)hi << 32) | lo;
}
__device__ __forceinline__ unsigned long long max_row16_u64(unsigned long long k) {
  unsigned long long o = dpp_u64<DPP_XOR1>(k);
  k = o > k ? o : k;
  o = dpp_u64<DPP_XOR2>(k);
  k = o > k ? o : k;
  o = dpp_u64<DPP_ROR4>(k);
  k = o > k ? o : k;
  o = dpp_u64<DPP_ROR8>(k);
  return o > k ? o : k;
}

// Order-preserving 64-bit argmax key: larger value first, then lower index.
__device__ __forceinline__ unsigned long long argmax_key(float v, int idx) {
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)u << 32) | (unsigned long long)(0xffffffffu - (uint32_t)idx);
}

// Final RMSNorm + tied lm_head GEMM (whole tiles per wave) + per-sequence argmax.
template <int MT>
__device__ __forceinline__ void phase_lm(BCtx& c, BLds<MT>& L, uint32_t epoch) {
  const BParams& p = *c.p;
  const int wave = wave_id(), lane = lane_id();
  int V0, V1, R0, R1;
  // vocabulary rows in multiples of 8: in the tiled lm_head the 8 rows of a
  // lane group are one 128-byte run of each block (a share of 501 rows would
  // split most 16-row tiles between two workgroups at odd offsets).
  share(VOCAB / 8, c.G, c.w, V0, V1);
  V0 *= 8;
  V1 *= 8;
  share(H, c.G, c.w, R0, R1);
  const int ntile = (V1 - V0 + 15) / 16;
  constexpr int UPT = H / (KS * 32);
  static_assert(UPT % 2 == 0, "unit pairs stay within a tile");
  const int my_tiles = ntile > wave ? (ntile - wave + NWAVE - 1) / NWAVE : 0;
  const int nunits = my_tiles * UPT;
  // every wave runs the same number of units (rounds of NWAVE tiles; a wave
  // without a tile in the last round streams nothing), so the rounds' LDS
  // barriers match
  const int all_units = (ntile + NWAVE - 1) / NWAVE * UPT;
  const rsrc_t rw = make_rsrc(p.lm, EMBED_BYTES);
  // the logits of a round: each wave's tile goes to LDS (the split-K area, idle
  // here), then every thread stores 32 contiguous bytes of one token's 64 rows,
  // so a token's logits leave in 256-byte runs instead of 64-byte pieces
  static_assert(sizeof(L.red) == (size_t)16 * MT * 64 * 4, "logit staging area");
  float (*stage)[64] = reinterpret_cast<float (*)[64]>(&L.red[0][0][0]);
  const rsrc_t rlog = make_rsrc(p.logits ? (const void*)p.logits : (const void*)p.lm,
                                p.logits ? (size_t)c.B * VOCAB * 4 : 0);
  // With one token tile the gate/up copy area (idle here) holds the logits of
  // the whole share instead: each wave writes its tiles there, with no
  // workgroup barrier per round, and the share leaves after the last round as
  // one contiguous run per token
  constexpr bool LGC = BLds<MT>::GW > 1;
  constexpr int LG_ROWS = 512, LG_STRIDE = LG_ROWS + 4;   // +4 floats: the lane groups' tokens on distinct banks
  static_assert(!LGC || sizeof(L.gw) >= sizeof(float) * 16 * MT * LG_STRIDE, "logit collection area");
  const bool lgc = LGC && V1 - V0 <= LG_ROWS;
  float* lgb = reinterpret_cast<float*>(&L.gw[0]);
  auto issue = [&](int u, u32x4(&wv)[KS]) {
    load_w<KS>(rw, p.tiled, u < nunits ? V0 + 16 * (wave + NWAVE * (u / UPT)) : V1, V1, H * 2, (u % UPT) * KS * 32, wv);
  };
  u32x4 wa[KS], wb[KS];
  issue(0, wa);
  issue(1, wb);
  trace_mark(c.s, 2 * xk(p.n_layers, 1) - 1);
  wait_h2(c, p.n_layers - 1);
  stage_norm<MT>(c, make_rsrc(c.xb(p.n_layers - 1, p.lay.h2), (size_t)c.B * H * 2), false, p.g_final, R0, R1, L);
  trace_mark(c.s, 2 * xk(p.n_layers, 1));
  prepare_next_launch(c, epoch);   // here the stores delay nothing
  f32x4 acc[MT];
  float best[MT][4];
  int bidx[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      best[mt][i] = -INFINITY;
      bidx[mt][i] = 0x7fffffff;
    }
  auto unit = [&](int u, u32x4(&wv)[KS]) {
    if (u % UPT == 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    mma_lds<MT>(L, (u % UPT) * KS * 32, wv, acc);
    issue(u + 2, wv);
    if (u % UPT == UPT - 1) {
      const int row = V0 + 16 * (wave + NWAVE * (u / UPT)) + (lane & 15);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = mt * 16 + (lane >> 4) * 4 + i;
          const float v = acc[mt][i];
          if (lgc) lgb[m * LG_STRIDE + (row - V0)] = v;   // row - V0 < 16 * 4 * ceil(ntile / 4) <= 512
          else stage[m][wave * 16 + (lane & 15)] = v;
          if (row < V1 && m < c.B && v > best[mt][i]) {   // a lane's rows ascend: keeps the lowest index among equal maxima
            best[mt][i] = v;
            bidx[mt][i] = row;
          }
        }
      if (lgc) return;
      lds_sync();
      {   // thread t: token t / 8, rows 8*(t % 8) .. +7 of the round
        const int t = tid(), m = t >> 3, r8 = (t & 7) * 8;
        const int row0 = V0 + 16 * NWAVE * (u / UPT) + r8;   // (V0, V1 and rows multiples of 8)
        const bool ok = m < c.B && row0 < V1;
        const uint32_t off = ok ? ((uint32_t)m * (uint32_t)VOCAB + (uint32_t)row0) * 4u : OOB;
        const float4 a = *reinterpret_cast<const float4*>(&stage[m < 16 * MT ? m : 0][r8]);
        const float4 b = *reinterpret_cast<const float4*>(&stage[m < 16 * MT ? m : 0][r8 + 4]);
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(a.x), __float_as_uint(a.y), __float_as_uint(a.z),
                                                     __float_as_uint(a.w)},
                                               rlog, (int)off, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(b.x), __float_as_uint(b.y), __float_as_uint(b.z),
                                                     __float_as_uint(b.w)},
                                               rlog, (int)(ok ? off + 16u : OOB), 0, 0);
      }
      lds_sync();   // the stage is rewritten in the next round
    }
  };
  for (int u = 0; u < all_units; u += 2) {
    unit(u, wa);
    unit(u + 1, wb);
  }
  // best per token over the 16 lanes of each lane row, then over the waves
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      unsigned long long k = bidx[mt][i] == 0x7fffffff ? 0ull : argmax_key(best[mt][i], bidx[mt][i]);
      k = max_row16_u64(k);
      if ((lane & 15) == 0) L.key[wave][mt * 16 + (lane >> 4) * 4 + i] = k;
    }
  __syncthreads();
  const int t = tid();
  if (t < c.B) {
    unsigned long long k = L.key[0][t];
#pragma unroll
    for (int w = 1; w < NWAVE; ++w) k = L.key[w][t] > k ? L.key[w][t] : k;
    if (k != 0ull)
      __hip_atomic_fetch_max(reinterpret_cast<unsigned long long*>(p.ws + BWS_KEY0 + (size_t)t * BWS_KEY_STRIDE), k,
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (lgc) {   // (the barrier above made every wave's tiles visible) token m's rows [V0, V1) in 16-byte pieces
    const int nq = (V1 - V0) / 4, q = t & 127;   // V0, V1 multiples of 8: nq <= 128
    for (int m = t >> 7; m < c.B; m += 2) {
      const float4 v = *reinterpret_cast<const float4*>(lgb + m * LG_STRIDE + 4 * q);
      const uint32_t off = q < nq ? ((uint32_t)m * (uint32_t)VOCAB + (uint32_t)(V0 + 4 * q)) * 4u : OOB;
      __builtin_amdgcn_raw_buffer_store_b128(
          u32x4{__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)}, rlog,
          (int)off, 0, 0);
    }
  }
}

// GFIX: the grid size when known at compile time (the per-phase work splits
// then divide by a constant); 0: gridDim.x.
template <int MT, int GFIX>
__global__ void __launch_bounds__(NT, 1) mk_batch_kernel(BParams p) {
  __shared__ BLds<MT> L;
  BCtx c;
  c.p = &p;
  uint32_t* ctrl = reinterpret_cast<uint32_t*>(p.ws);
  c.s.err = ctrl + C_ERR;
  c.s.timeout = p.timeout_ticks;
  c.s.trace = p.trace ? p.trace + (size_t)blockIdx.x * MK_TRACE_SLOTS : nullptr;
  trace_mark(c.s, 0);
  c.G = GFIX ? GFIX : (int)gridDim.x;
  c.w = blockIdx.x;
  c.B = p.batch;
  c.prefill = (p.flags & MK_FLAG_PREFILL) != 0;
  const int t = tid();
  const uint32_t epoch = __hip_atomic_load(ctrl + C_EPOCH, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  int tok = 0, ps = 0;
  if (t < c.B) {
    ps = p.pos[t];
    tok = p.tokens ? p.tokens[t] : 0;
  }
  // the first layer's first QKV weight unit depends on nothing: issued behind
  // the control, position and token loads, so that the setup below and the
  // plan run while it lands
  u32x4 wv[KS];
  qkv_first_unit<MT>(c, 0, wv);
  const size_t cset = bws_cnt_set(p.max_batch);
  uint8_t* cnt0 = p.cnt;
  c.hcnt = cnt0 + (size_t)(epoch & 1u) * cset;
  c.acnt = reinterpret_cast<uint32_t*>(c.hcnt + HCNT_BYTES);
  c.dcnt = c.acnt + (size_t)MK_MAX_LAYERS * p.max_batch * NKV;
  c.dng = c.G / DN_KQ;
  c.drpg = c.dng > 0 ? H / c.dng : 0;
  // (batch 8 measured slower with it: there act is small and the extra hand-over costs more)
  c.dpair = (H + c.G - 1) / c.G <= 8;
  c.d2 = MT == 2 && c.G % DN_KQ == 0 && c.dng <= DN_MAX && c.dng * c.drpg == H && c.drpg % 16 == 0 &&
         c.drpg <= RES_MAX;
  c.sset = p.xch + p.lay.sent_base + (size_t)(epoch & 1u) * p.lay.sset;
  c.cnt_other = reinterpret_cast<uint32_t*>(cnt0 + (size_t)((epoch + 1u) & 1u) * cset);
  c.cnt_words = (int)(cset / 4);
  if (t < c.B) {
    L.pos[t] = ps;
    L.tok[t] = tok < 0 ? 0 : (tok >= VOCAB ? VOCAB - 1 : tok);
  }
  lds_sync();   // (not __syncthreads: that would also wait for the weight unit)
  // every sequence's position in range (and consecutive in a prefill step):
  // lane b checks sequence b, each wave the whole batch
  bool pos_ok, run_ok;
  {
    const int lane = lane_id();
    const int ps = lane < c.B ? L.pos[lane] : 0;
    pos_ok = __ballot(lane < c.B && !(ps >= 0 && ps < p.s_max && ps < p.rope_rows)) == 0ull;
    run_ok = __ballot(lane < c.B && c.prefill && ps != L.pos[0] + lane) == 0ull;
  }
  if (!pos_ok && blockIdx.x == 0 && t == 0)
    __hip_atomic_fetch_or(c.s.err, MK_DEVERR_POS, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (!run_ok && blockIdx.x == 0 && t == 0)
    __hip_atomic_fetch_or(c.s.err, MK_DEVERR_PREFILL, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  pos_ok = pos_ok && run_ok;
  if (MT == 2 && pos_ok) {
    plan_and_rope<MT>(c, L);
    lds_sync();
  }

  if (pos_ok) {
    phase_qkv<MT, true>(c, 0, L, wv);
    for (int li = 0; li < p.n_layers; ++li) {
      if constexpr (MT == 2) {
        // two token tiles: each layer reads the parameters and the workgroup
        // index afresh through opaque copies, so fewer values stay live in
        // scalar registers across the layer loop (93 spilled SGPRs instead of
        // 247: C5 +0.4%; the one-tile kernel ran 1% slower with it)
        c.w = opaque_s(c.w);
        c.p = opaque_params();
      }
      phase_attn<MT>(c, li, L);
      GuCopy guc;
      gu_copy_init<MT>(c, li, L, guc);
      phase_o<MT>(c, li, L, guc);
      phase_gu<MT>(c, li, L, guc);
      if (c.d2) {
        phase_down2d<MT>(c, li, L);
      } else if constexpr (MT == 1) {
        if (c.dpair && c.B <= 8) phase_down_pair<MT>(c, li, L);
        else phase_down<MT>(c, li, L);
      } else {
        phase_down<MT>(c, li, L);
      }
      if (li + 1 < p.n_layers) {
        u32x4 wn[KS];
        phase_qkv<MT, false>(c, li + 1, L, wn);
      }
    }
    if (p.do_lm) phase_lm<MT>(c, L, epoch);
  }
  if (!p.do_lm || !pos_ok) prepare_next_launch(c, epoch);   // (the lm_head phase does it otherwise)

  // ---- exit: the last workgroup out publishes the tokens and advances the epoch ----
  trace_mark(c.s, MK_TRACE_SLOTS - 1);
  wait_mem();
  __syncthreads();
  if (t == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(ctrl + C_EXIT, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    L.flag = prev == (uint32_t)(c.G - 1);
  }
  __syncthreads();
  if (!L.flag) return;
  if (t == 0) {
    ctrl[C_EXIT] = 0u;
    ctrl[C_EPOCH] = epoch + 1u;
  }
  if (pos_ok && t < c.B) {   // thread b: sequence b (one memory round trip, not B in a row)
    const int b = t;
    if (p.do_lm) {
      unsigned long long* kp = reinterpret_cast<unsigned long long*>(p.ws + BWS_KEY0 + (size_t)b * BWS_KEY_STRIDE);
      const unsigned long long key = __hip_atomic_load(kp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *kp = 0ull;
      if (p.next_token) p.next_token[b] = (int32_t)(0xffffffffu - (uint32_t)(key & 0xffffffffull));
    }
    if (p.flags & MK_FLAG_ADVANCE) p.pos[b] = L.pos[b] + 1;
  }
}

}  // namespace

#ifdef MK_BATCH_TILE2

namespace mk {
// The two-tile kernel of this translation unit for a grid of `grid` workgroups.
const void* batch_kernel_tile2(int grid) {
  return grid == 256 ? reinterpret_cast<const void*>(mk_batch_kernel<2, 256>)
                     : reinterpret_cast<const void*>(mk_batch_kernel<2, 0>);
}
}  // namespace mk

#else

namespace {
struct BDev {
  int ready;
  int status;
  char msg[256];
};
BDev g_bdev[64];
std::mutex g_bdev_mu;
}  // namespace

namespace mk {

// The batched kernel for `batch` tokens on a grid of `grid` workgroups: one
// 16-row MFMA tile up to 16 tokens, two above (mk_batch_tile2.hip); MI355X's
// 256 CUs get the instantiations with the grid size fixed at compile time.
const void* batch_kernel_for(int batch, int grid) {
  if (batch > 16) return batch_kernel_tile2(grid);
  return grid == 256 ? reinterpret_cast<const void*>(mk_batch_kernel<1, 256>)
                     : reinterpret_cast<const void*>(mk_batch_kernel<1, 0>);
}

int batch_device_check(int dev, char* msg, size_t msg_len) {
  if (dev < 0 || dev >= 64) {
    snprintf(msg, msg_len, "device index %d out of range", dev);
    return MK_ERR_DEVICE;
  }
  std::lock_guard<std::mutex> lk(g_bdev_mu);
  BDev& d = g_bdev[dev];
  if (!d.ready) {
    int cus = 0, nb1 = 0, nb2 = 0;
    d.status = MK_OK;
    d.msg[0] = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb1, batch_kernel_for(1, cus), NT, 0) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb2, batch_kernel_for(17, cus), NT, 0) != hipSuccess) {
      d.status = MK_ERR_HIP;
      snprintf(d.msg, sizeof(d.msg), "device query for the batched kernel failed on device %d", dev);
    } else if (nb1 < 1 || nb2 < 1) {
      d.status = MK_ERR_DEVICE;
      snprintf(d.msg, sizeof(d.msg), "batched kernel cannot be resident on a CU (occupancy %d / %d)", nb1, nb2);
    } else if (cus < B_MIN_GRID) {
      d.status = MK_ERR_DEVICE;
      snprintf(d.msg, sizeof(d.msg), "batched kernel needs >= %d CUs, device %d has %d", B_MIN_GRID, dev, cus);
    }
    d.ready = 1;
  }
  if (d.status != MK_OK) snprintf(msg, msg_len, "%s", d.msg);
  return d.status;
}

hipError_t batch_launch(const mk_weights* w, const mk_step_args* a, uint8_t* xch, uint8_t* cnt, int max_batch,
                        int grid, unsigned long long timeout_ticks) {
  BParams kp;
  memset(&kp, 0, sizeof(kp));
  kp.w_qkv = static_cast<const uint16_t*>(w->w_qkv);
  kp.w_o = static_cast<const uint16_t*>(w->w_o);
  kp.w_gu = static_cast<const uint16_t*>(w->w_gu);
  kp.w_d = static_cast<const uint16_t*>(w->w_down);
  kp.embed = static_cast<const uint16_t*>(w->embed);
  kp.lm = kp.embed;
  if (w->t_qkv && w->t_o && w->t_gu && w->t_down && w->t_embed) {
    kp.tiled = 1;
    kp.w_qkv = static_cast<const uint16_t*>(w->t_qkv);
    kp.w_o = static_cast<const uint16_t*>(w->t_o);
    kp.w_gu = static_cast<const uint16_t*>(w->t_gu);
    kp.w_d = static_cast<const uint16_t*>(w->t_down);
    kp.lm = static_cast<const uint16_t*>(w->t_embed);
  }
  kp.g_final = static_cast<const uint16_t*>(w->norm_final);
  kp.rope = static_cast<const uint16_t*>(w->rope);
  for (int i = 0; i < a->n_layers; ++i) {
    kp.kc[i] = static_cast<uint16_t*>(a->k_cache[i]);
    kp.vc[i] = static_cast<uint16_t*>(a->v_cache[i]);
  }
  kp.tokens = a->tokens;
  kp.hidden_in = static_cast<const uint16_t*>(a->hidden_in);
  kp.pos = a->pos;
  kp.hidden_out = static_cast<uint16_t*>(a->hidden_out);
  kp.logits = a->logits;
  kp.next_token = a->next_token;
  kp.ws = static_cast<uint8_t*>(a->workspace);
  kp.xch = xch;
  kp.cnt = cnt;
  kp.lay.init(max_batch);
  kp.batch = a->batch;
  kp.max_batch = max_batch;
  kp.first_layer = a->first_layer;
  kp.n_layers = a->n_layers;
  kp.s_max = a->s_max;
  kp.rope_rows = w->rope_rows;
  kp.do_lm = (a->logits != nullptr || a->next_token != nullptr) ? 1 : 0;
  kp.flags = a->flags;
  kp.timeout_ticks = timeout_ticks;
  kp.trace = static_cast<unsigned long long*>(a->trace);
  void* args[] = {&kp};
  const void* fn = batch_kernel_for(a->batch, grid);
  const hipStream_t st = static_cast<hipStream_t>(a->stream);
  return (a->flags & MK_FLAG_COOPERATIVE) ? hipLaunchCooperativeKernel(fn, dim3(grid), dim3(NT), args, 0, st)
                                          : hipLaunchKernel(fn, dim3(grid), dim3(NT), args, 0, st);
}

}  // namespace mk

#endif  // MK_BATCH_TILE2
