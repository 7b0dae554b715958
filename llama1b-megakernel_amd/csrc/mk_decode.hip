// mk_decode.hip — Llama-3.2-1B token-generation megakernel for MI355X (gfx950).
//
// One kernel launch runs a whole decode step: for every decoder layer
//   QKV  : RMSNorm(h) -> [Wq;Wk;Wv] GEMV -> RoPE -> q and the fresh K/V row,
//          which is also written in place into the caches at row pos
//                                                              (attention.py:69-245, 450-492)
//   ATTN : GQA attention of the 32 q heads over K/V rows [0, pos], split over
//          the KV length; the first split of each kv head merges the partial
//          (max, sum, PV) of all splits of that head          (attention.py:303-399)
//   O    : Wo GEMV + residual                                  (attention.py:409-448,
//                                                                transformer_llama.py:68-70)
//   GU   : RMSNorm(h1) -> gate/up GEMV -> silu(g)*u            (mlp.py:72-157)
//   DOWN : Wd GEMV + residual                                  (mlp.py:159-192,
//                                                                transformer_llama.py:82-84)
// then, optionally, the final RMSNorm, the tied lm_head GEMV and the greedy argmax.
//
// Design for CDNA4:
//   * one 256-thread workgroup (4 wave64s, one per SIMD) per CU, grid = #CUs,
//     occupancy 1, so all workgroups are resident together (a plain launch on
//     an idle device, or a cooperative launch on request);
//   * no grid barriers. Phases hand their results over through per-layer
//     exchange buffers that hold a sentinel (all-ones bits: a NaN the kernel
//     never stores) until written. A producer stores its results with
//     device-scope (sc1) stores and moves on; a consumer polls the buffer itself
//     with device-scope loads until no sentinel is left. The data is its own
//     ready flag, so a hand-over costs one store propagation plus one load
//     round trip: no wait for store completion, no atomic counter, no second
//     read after a flag. Two buffer sets alternate between launches (an epoch
//     counter in the workspace picks the set): launch n works in set n&1 and
//     refills set (n+1)&1 with the sentinel; nothing reads that set before
//     launch n+1, and kernel boundaries order the two launches. The sets live
//     in uncached device memory: an all-to-all hand-over under a full HBM
//     weight stream measured 3.8 us there against 6 us in L2-cached memory;
//   * weights stream once from HBM through bounds-checked buffer loads (16 B
//     per lane, fully coalesced 1 KiB per wave per load, non-temporal); rows
//     past a wave's share are out-of-range offsets that return zero without a
//     memory access, so the software pipeline has no branches around its loads;
//   * before polling for its input each wave has already issued the first
//     ring of the phase's weight loads (they do not depend on the
//     activations), so the hand-over latency overlaps HBM traffic;
//   * a CU's vector memory operations complete in order, so a hand-over poll
//     or result store waits for every load the CU issued before it; each
//     layer's bytes are therefore placed in the windows where the CU would
//     otherwise wait or compute, with only about a hand-over latency's worth
//     ahead of each poll: during the layer-input and attention hand-overs each
//     wave copies the first 4 gate/up pairs of its GU share (32 KiB) straight
//     from HBM into LDS (buffer loads with the LDS bit), a few 1 KiB chunks
//     per poll round; the O workgroups load 2 more gate/up pairs into
//     registers before the attention-output wait; the first 8 KiB of each
//     wave's down row are loaded during the gate/up dot products; attention
//     items issue their cached K/V rows before they wait for q; the
//     workgroups with attention items get no O rows, so h1 does not wait for
//     the last merge;
//   * GEMVs are bf16 x bf16 -> fp32 with v_dot2_f32_bf16, reduced across the
//     wave with DPP row operations and four lane reads (bs=1 is
//     bandwidth-bound: no MFMA);
//   * every workgroup stages the layer input and h1 in LDS, where the
//     residual adds read them.
#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "mk.h"
#include "mk_batch.h"
// The single-step instantiations of the kernel are compiled in a translation
// unit of their own, mk_decode_step.hip, which includes this file with
// MK_DECODE_STEP_TU defined: there the thread index is opaque to the optimiser
// (tid() in mk_common.h), which made one-layer launches 1.5% faster; the
// decode loop's instantiation, compiled here with the plain index, ran 0.45%
// slower with it.
#ifdef MK_DECODE_STEP_TU
#define MK_OPAQUE_TID 1
#endif
#include "mk_common.h"
#include "mk_prefill.h"

namespace {

using namespace mk;

// Tuning constants (values measured best on MI355X; the alternatives and their
// results are recorded with the design notes).
constexpr int ATT_MAX_SPLIT = 8;           // KV-length splits per kv head (attention work items)
constexpr int ATT_RD = 4;                  // rounds of 32 rows per attention group
constexpr int GU_LDS_PAIRS = 4;            // gate/up pairs per wave copied HBM -> LDS ahead of the GU phase
// 1 KiB chunks of that copy issued per poll round of the layer-input wait and
// of the attention-output wait
constexpr int GU_LDS_STEP_QKV = 8, GU_LDS_STEP_O = 6;
constexpr int O_RING = 4;                  // O rows per wave in the register ring
// Gate/up pairs per wave (after the LDS ones) loaded into registers before the
// attention-output wait on workgroups with O rows, so that the h1 wait queues
// behind fewer weight loads; the other GU_RING pairs of the wave's first eight
// are issued after the O projection.
constexpr int GU_EARLY = 2;
constexpr int GU_RING = 4 - GU_EARLY;
// 1 KiB chunks of the wave's first down-projection row loaded before the
// gate/up dot products (they land while those run, so the act store that
// queues behind them is not delayed, and HBM is not idle meanwhile).
constexpr int D_EARLY = 8;
constexpr int LM_RING = 8;                 // lm_head rows per wave in the register ring (4 KiB each)
constexpr int MIN_GRID = 32;
constexpr int MAX_GRID = 1024;


// Workspace (bytes, batch 1): a control block. The two sets of exchange buffers
// live in a separate uncached area (SET_BYTES each) tied to the workspace.
constexpr size_t CTRL_BYTES = 256;
constexpr int C_EXIT = 0, C_ERR = 1, C_EPOCH = 2;   // u32 words of the control block
constexpr int C_STICKY = 3;   // allocation-free scratch only: error bits of every faulted step since the last read
constexpr size_t C_KEY_BYTE = 128;                  // u64 argmax key (a decode loop alternates it
                                                    // with C_KEY_BYTE + 64 by step parity)
// Decode loop (several steps in one launch): step-barrier sub-counters, one
// 128-byte line each, in the workspace's exchange area after the two sets.
constexpr int STEP_LINES = 32;
constexpr size_t STEP_LINE = 128;
constexpr size_t STEP_CNT_BYTES = (size_t)STEP_LINES * STEP_LINE;
// Exchange buffers of one layer; each region starts on a 256-byte boundary.
constexpr size_t X_QKV = 0;                                 // bf16 q[2048] | k[512] | v[512]
constexpr size_t X_K = (size_t)NQ * HD * 2, X_V = X_K + (size_t)NKV * HD * 2;   // within X_QKV
constexpr size_t X_ATT = X_QKV + (size_t)(NQ + 2 * NKV) * HD * 2;  // bf16 [2048] attention output
constexpr size_t X_H1 = X_ATT + H * 2;                      // bf16 [2048] h + attn
constexpr size_t X_ACT = X_H1 + H * 2;                      // bf16 [8192] silu(gate) * up
constexpr size_t X_H2 = X_ACT + INTER * 2;                  // bf16 [2048] layer output
constexpr size_t X_PART = X_H2 + H * 2;                     // fp32 [kv head][split][m(4) l(4) o(4x64)]
constexpr size_t X_LAYER = X_PART + (size_t)NKV * ATT_MAX_SPLIT * PART_FLOATS * 4;
constexpr size_t SET_BYTES = (size_t)MK_MAX_LAYERS * X_LAYER;
constexpr size_t WS_BYTES = CTRL_BYTES;   // the exchange sets live in a separate uncached area
static_assert(X_ATT % 256 == 0 && X_PART % 256 == 0 && X_LAYER % 256 == 0, "exchange regions must be aligned");


// ---------------------------------------------------------------------------
// Kernel parameters
// ---------------------------------------------------------------------------
struct KParams {
  const uint16_t* w_qkv;
  const uint16_t* w_o;
  const uint16_t* w_gu;
  const uint16_t* w_d;
  const uint16_t* embed;
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
  uint8_t* xch;   // exchange sets (uncached device memory)
  int first_layer;
  int n_layers;
  int s_max;
  int rope_rows;
  int do_lm;
  int noalloc;   // control block and exchange sets in the library's static scratch
  uint32_t flags;
  unsigned long long timeout_ticks;
  unsigned long long* trace;
  int n_steps;                      // decode steps of this launch (a greedy loop when > 1)
  int32_t* tokens_out;              // [n_steps] each step's greedy token, or NULL
  unsigned long long* step_clock;   // [n_steps + 1] device wall clock at the step boundaries, or NULL
  uint32_t* step_cnt;               // loop: the step-barrier sub-counters (STEP_LINES lines)
};

// ---------------------------------------------------------------------------
// Row streams: a wave's share of a GEMV, software pipelined through a ring of
// RING rows held in VGPRs. Row r of the wave starts at byte off0 + r*stride;
// the lane reads 16 bytes at i*1024 + lane*16 for chunk i < KCH, i.e. the
// elements i*512 + lane*8 .. +7 of the row. Loads for rows >= n use OOB and
// return zero without touching memory.
// ---------------------------------------------------------------------------
template <int RING, int KCH>
struct RowStream {
  u32x4 buf[RING][KCH];
  rsrc_t rs;
  uint32_t off0, stride;
  int n;

  __device__ __forceinline__ uint32_t row_off(int r) const {
    return r < n ? off0 + (uint32_t)r * stride : OOB;
  }
  // Chunks i < skip read nothing (zero): the caller has loaded them already.
  __device__ __forceinline__ void issue(int slot_row, u32x4 (&dst)[KCH], int skip = 0) const {
    const uint32_t o = row_off(slot_row) + (uint32_t)lane_id() * 16u;
#pragma unroll
    for (int i = 0; i < KCH; ++i) dst[i] = ld_stream(rs, i < skip ? OOB : o + (uint32_t)i * 1024u);
  }
  __device__ __forceinline__ void start(rsrc_t r, uint32_t o0, uint32_t st, int count, int skip0 = 0) {
    rs = r;
    off0 = o0;
    stride = st;
    n = count;
#pragma unroll
    for (int j = 0; j < RING; ++j) issue(j, buf[j], j == 0 ? skip0 : 0);
  }
  // When n <= RING: the per-lane partials of all RING slots (rows >= n read
  // zero, so their partials are 0), with no refill loads.
  template <class DotF, class T>
  __device__ __forceinline__ void dots(DotF&& dotf, T (&part)[RING]) const {
#pragma unroll
    for (int j = 0; j < RING; ++j) part[j] = dotf(buf[j]);
  }
  // dotf(buf) -> partial (per lane); emit(r, partial) for each valid row r.
  // The last RING refills are past the rows (out of range, nothing read); they
  // are drained here, so that no later code that reuses the ring's registers
  // has to wait for every memory operation issued meanwhile (result stores
  // and background copies included).
  template <class DotF, class EmitF>
  __device__ __forceinline__ void run(DotF&& dotf, EmitF&& emit) {
    for (int base = 0; base < n; base += RING) {
#pragma unroll
      for (int j = 0; j < RING; ++j) {
        const int r = base + j;
        auto part = dotf(buf[j]);
        issue(r + RING, buf[j]);
        if (r < n) emit(r, part);
      }
    }
    wait_mem();
  }
};

// The wave's rows of a workgroup share [lo, hi): lo + wave + 4*j (QKV), or
// a contiguous block (the other GEMVs) so the wave stores its results with one
// instruction and streams contiguous memory.
__device__ __forceinline__ int wave_count(int lo, int hi) {
  const int n = hi - lo - wave_id();
  return n > 0 ? (n + NWAVE - 1) / NWAVE : 0;
}
struct Span {
  int lo, n;
};
__device__ __forceinline__ Span wave_span(int lo, int hi) {
  int a, b;
  share(hi - lo, NWAVE, wave_id(), a, b);
  return Span{lo + a, b - a};
}

// A wave's background copy of `total` contiguous 1 KiB chunks of weights
// (starting at byte off0 of resource rs) straight from HBM into its own LDS
// region, issued a few chunks at a time; chunk k lands at dst + k*1024.
// The wave waits for them with s_waitcnt vmcnt before reading the region.
struct LdsPrefetch {
  rsrc_t rs;
  uint32_t off0, stride;   // row r of the copy starts at off0 + r*stride
  int kch;                 // 1 KiB chunks per row
  int total, next;
  uint8_t* dst;
  __device__ __forceinline__ void init(rsrc_t r, uint32_t o0, uint32_t st, int chunks_per_row, int rows,
                                       uint8_t* lds) {
    rs = r;
    off0 = o0;
    stride = st;
    kch = chunks_per_row;
    total = rows * chunks_per_row;
    next = 0;
    dst = lds;
  }
  __device__ __forceinline__ void issue(int n) {
    const int end = min(total, next + n);
    for (; next < end; ++next)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs, (__attribute__((address_space(3))) void*)(dst + next * 1024), 16,
          off0 + (uint32_t)(next / kch) * stride + (uint32_t)(next % kch) * 1024u + (uint32_t)lane_id() * 16u, 0, 0,
          AUX_NT);
  }
  // Exactly K copy instructions, a fixed count, so that a wait for loads
  // issued just before them can count past them (vector loads complete in
  // order): chunks beyond the copy go to `spare`, a 1 KiB LDS area nobody
  // reads, from an out-of-range offset that reads no memory.
  template <int K>
  __device__ __forceinline__ void issue_fixed(uint8_t* spare) {
    const int nx = __builtin_amdgcn_readfirstlane(next);
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int ck = nx + k;
      const bool real = ck < total;
      uint8_t* d = real ? dst + ck * 1024 : spare;
      const uint32_t o =
          real ? off0 + (uint32_t)(ck / kch) * stride + (uint32_t)(ck % kch) * 1024u + (uint32_t)lane_id() * 16u : OOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)d, 16, o, 0, 0, AUX_NT);
    }
    next = min(total, nx + K);
  }
};

// GU pairs [0, GU_LDS_PAIRS) of this wave's share, HBM -> L.gu[wave] (pair j at j*8 KiB).
struct GuPrefetch : LdsPrefetch {
  __device__ __forceinline__ void start(const uint16_t* w_gu_layer, Span gp, uint8_t* region) {
    init(make_rsrc(w_gu_layer, GU_LAYER_BYTES), (uint32_t)gp.lo * (2 * H * 2), 2 * H * 2, 8,
         min(gp.n, GU_LDS_PAIRS), region);
  }
};

// Gate/up pairs [n_lds, n_lds + GU_EARLY) of the wave's share in registers
// (pairs past the share read zero from out-of-range offsets).
struct GuEarly {
  u32x4 buf[GU_EARLY > 0 ? GU_EARLY : 1][8];
  __device__ __forceinline__ void issue(const uint16_t* w_gu_layer, Span sp, int n_lds) {
    const rsrc_t r = make_rsrc(w_gu_layer, GU_LAYER_BYTES);
#pragma unroll
    for (int j = 0; j < GU_EARLY; ++j) {
      const int row = n_lds + j;
      const uint32_t o = (row < sp.n ? (uint32_t)(sp.lo + row) * (2 * H * 2) : OOB) + (uint32_t)lane_id() * 16u;
#pragma unroll
      for (int i = 0; i < 8; ++i) buf[j][i] = ld_stream(r, o + (uint32_t)i * 1024u);
    }
  }
};

// ---------------------------------------------------------------------------
// The megakernel
// ---------------------------------------------------------------------------
struct Lds {
  __attribute__((aligned(16))) uint16_t x[H];       // layer input (raw): QKV input, O residual
  __attribute__((aligned(16))) uint16_t h1[H];      // h1 (raw): GU input, DOWN residual
  __attribute__((aligned(16))) uint16_t v[INTER];   // staged GEMV input: attention output / act
  __attribute__((aligned(16))) uint16_t q[GQA * HD + 2 * HD];  // attention: 4 q heads | fresh k | fresh v
  float val[128];                                    // QKV dot products of this workgroup
  __attribute__((aligned(16))) uint16_t rope[2 * HD];  // RoPE row of this step's position: cos | sin
  AttnShared att;
  float best[NWAVE];
  int bidx[NWAVE];
  int last;
  __attribute__((aligned(16))) uint8_t gu[NWAVE][GU_LDS_PAIRS * 8192];   // GU pairs copied ahead (per wave)
  __attribute__((aligned(16))) uint8_t spare[1024];                       // target of padding copies
};

struct Ctx {
  const KParams* p;
  Sync s;
  int G, w;
  int pos;
  int n_rows;            // KV rows attended: pos + 1
  const uint16_t* x_in;  // input of the first layer (embedding row or hidden_in): final data
  uint8_t* set;          // this launch's exchange buffers
  // Work split, the same for every layer (computed once per launch: the
  // divisions by the grid size are not cheap on the GPU)
  int P0, P1;            // QKV RoPE pairs of the workgroup
  int qkv_n;             // QKV rows of this wave: 2*P0 + wave + 4*j, j < qkv_n
  int nsplit;            // attention: KV splits per kv head
  Span o_rows;           // this wave's O rows (empty on workgroups with attention items)
  bool has_o;            // the workgroup has O rows
  Span gu_pairs;         // this wave's gate/up pairs
  Span d_rows;           // this wave's down-projection rows
  bool loop;             // a decode loop (the kernel's LOOP instantiation): cache rows by device-scope stores

  __device__ __forceinline__ uint16_t* xb(int li, size_t off) const {
    return reinterpret_cast<uint16_t*>(set + (size_t)li * X_LAYER + off);
  }
  __device__ __forceinline__ float* part(int li) const {
    return reinterpret_cast<float*>(set + (size_t)li * X_LAYER + X_PART);
  }
};

// Trace exchange index of phase `ph` (1 QKV, 2 ATTN, 3 O, 4 GU, 5 DOWN) of run-layer li.
__device__ __forceinline__ int xk(int li, int ph) { return 5 * li + ph; }

// The wave's QKV weight rows of run-layer li: rows 2*P0 + wave + 4*j, j < n.
__device__ __forceinline__ void qkv_rows(const Ctx& c, int li, rsrc_t& r, uint32_t& off0, int& n) {
  const KParams& p = *c.p;
  r = make_rsrc(p.w_qkv + (size_t)(p.first_layer + li) * QKV_ROWS * H, QKV_LAYER_BYTES);
  off0 = (uint32_t)(2 * c.P0 + wave_id()) * (H * 2);
  n = c.qkv_n;
}

// QKV phase of run-layer li: RMSNorm, GEMV, RoPE; q and the fresh K/V row to
// the exchange buffer, the K/V row also into the caches. idle() runs between
// the polls for the layer input.
// The wave's QKV weight ring of run-layer li, issued (the caller issues it
// before phase_qkv; the first layer's at kernel start).
__device__ __forceinline__ void qkv_ring(const Ctx& c, int li, RowStream<4, 4>& rs) {
  rsrc_t wr;
  uint32_t woff;
  int wn;
  qkv_rows(c, li, wr, woff, wn);
  rs.start(wr, woff, NWAVE * H * 2, wn);
}

// rs: this layer's ring, already issued. pre_sync() runs just before the
// workgroup barrier that follows the wait for the layer input.
template <class Idle, class PreSync>
__device__ __forceinline__ void phase_qkv(Ctx& c, int li, Lds& L, Idle&& idle, RowStream<4, 4>& rs,
                                          PreSync&& pre_sync) {
  const KParams& p = *c.p;
  const int wave = wave_id();
  const int P0 = c.P0, P1 = c.P1;
  const int wn = c.qkv_n;
  trace_mark(c.s, 2 * xk(li, 1) - 1);
  if (li == 0) stage_vec<1>(c.s, c.x_in, false, L.x);
  else stage_vec<1>(c.s, c.xb(li - 1, X_H2), true, L.x, idle);
  pre_sync();
  lds_sync();
  trace_mark(c.s, 2 * xk(li, 1));
  u32x4 xs[4];
  lds_x2048(L.x, xs);
  rmsnorm2048(xs, nullptr);
  auto dotf = [&](const u32x4(&wv)[4]) { return dot2048(wv, xs); };
  if (wn <= 4) {   // all rows in the ring: one transposed reduction
    float pt[4];
    rs.dots(dotf, pt);
    const float v = reduce_rows<4>(pt);
    const int r = lane_id() >> 4;
    if ((lane_id() & 15) == 0 && r < wn) L.val[wave + NWAVE * r] = v;
  } else {
    rs.run(dotf, [&](int r, float part) {
      const float v = wave_sum(part);
      if (lane_id() == 0) L.val[wave + NWAVE * r] = v;
    });
  }
  lds_sync();
  const uint16_t* rrow = L.rope;
  uint16_t* xq = c.xb(li, X_QKV);
  uint16_t* const kcl = p.kc[li];
  uint16_t* const vcl = p.vc[li];
  for (int lp = tid(); lp < P1 - P0; lp += NT) {
    const int pr = P0 + lp, d = pr & 31;
    const float a = rbf(L.val[2 * lp]), b = rbf(L.val[2 * lp + 1]);
    if (pr < Q_PAIRS) {
      const u32x4 o = rope_pair(a, b, rrow, d);
      uint16_t* dst = xq + (pr >> 5) * HD + d;
      st_dev(dst, o.x);
      st_dev(dst + 32, o.y);
    } else {
      const bool is_k = pr < Q_PAIRS + K_PAIRS;
      const int kh = (pr - Q_PAIRS - (is_k ? 0 : K_PAIRS)) >> 5;
      const u32x4 o = is_k ? rope_pair(a, b, rrow, d) : u32x4{f2bf(a), f2bf(b), 0u, 0u};
      uint16_t* dst = xq + (is_k ? X_K : X_V) / 2 + kh * HD + d;
      st_dev(dst, o.x);
      st_dev(dst + 32, o.y);
      // the cache row: read by later launches (a plain store), or, in a decode
      // loop, by the next step of this launch on any XCD (a device-scope store)
      uint16_t* crow = (is_k ? kcl : vcl) + ((size_t)kh * p.s_max + c.pos) * HD + d;
      if (c.loop) {
        st_dev(crow, o.x);
        st_dev(crow + 32, o.y);
      } else {
        crow[0] = (uint16_t)o.x;
        crow[32] = (uint16_t)o.y;
      }
    }
  }
  trace_done(c.s, li, 0);
}

// ATTN phase: the workgroup's attention items (kv head, KV split). The KV
// rows form ng = ceil(n_rows / 32) groups of 32; split sp of a head takes the
// groups [sp * ng / nsplit, (sp + 1) * ng / nsplit): one group per split below
// 256 rows, else eight splits whose sizes differ by at most one group. (Eight
// splits at every length from 256 rows on: with whole splits of a fixed size
// the count drops to 6 or 7 over about half of the 384..1023 positions, and
// those steps took 5-7 us longer.)
__device__ __forceinline__ void phase_attn(Ctx& c, int li, Lds& L) {
  const int nsplit = c.nsplit;
  const int nitems = NKV * nsplit;
  const int lane = lane_id();
  for (int it = c.w; it < nitems; it += c.G) {
    const int h = it / nsplit, sp = it % nsplit;
    const int ng = (c.n_rows + 31) >> 5;
    const int j0 = 32 * (sp * ng / nsplit), j1 = min(32 * ((sp + 1) * ng / nsplit), c.n_rows);
    const bool fresh = c.pos >= j0 && c.pos < j1;
    // the item's cached rows do not depend on this step: their first group is issued before the wait for q
    AttnRows ar;
    ar.init(c.p->kc[li] + (size_t)h * c.p->s_max * HD, c.p->vc[li] + (size_t)h * c.p->s_max * HD, c.p->s_max, j0,
            min(j1, c.pos));
    AttnGroupT<ATT_RD> g0;
    ar.load(0, g0);
    if (it == c.w) trace_mark(c.s, 2 * xk(li, 2) - 1);
    if (wave_id() == 0) {
      // q of heads 4h..4h+3 (512 B, lanes 0-31), the fresh K row (lanes 32-39) and V row (40-47)
      const rsrc_t r = make_rsrc(c.xb(li, X_QKV), X_ATT - X_QKV);
      uint32_t off[1];
      off[0] = lane < 32 ? (uint32_t)(h * GQA * HD * 2 + lane * 16)
             : lane < 40 ? (fresh ? (uint32_t)(X_K + h * HD * 2 + (lane - 32) * 16) : OOB)
             : lane < 48 ? (fresh ? (uint32_t)(X_V + h * HD * 2 + (lane - 40) * 16) : OOB)
                         : OOB;
      u32x4 v[1];
      poll_bf16<1>(c.s, r, off, v);
      if (lane < 48) *reinterpret_cast<u32x4*>(L.q + lane * 8) = v[0];
    }
    lds_sync();
    if (it == c.w) trace_mark(c.s, 2 * xk(li, 2));
    attn_item(ar, g0, L.q, fresh, c.part(li) + ((size_t)h * ATT_MAX_SPLIT + sp) * PART_FLOATS, L.att);
    if (sp == 0)
      attn_merge_head<true, ATT_MAX_SPLIT>(c.s, c.part(li) + (size_t)h * ATT_MAX_SPLIT * PART_FLOATS, nsplit,
                                           c.xb(li, X_ATT) + h * GQA * HD);
    trace_done(c.s, li, 1);
  }
}

// GFIX: the grid size when it is known at compile time (the work splits then
// divide by a constant: multiply and shift instead of a ~20-instruction
// division each, ~1.8 us of the prologue at one wave per SIMD); 0: gridDim.x.
// LOOP: the decode loop's instantiation (p.n_steps steps, the step barrier,
// tokens_out / step_clock); without it the kernel is one step and carries
// none of that code.
template <int GFIX, bool LOOP>
__global__ void __launch_bounds__(NT, 1) mk_decode_kernel(KParams p) {
  __shared__ Lds L;

  Ctx c;
  c.p = &p;
  c.loop = LOOP;
  const int n_steps = LOOP ? p.n_steps : 1;
  uint32_t* ctrl = reinterpret_cast<uint32_t*>(p.ws);
  c.s.err = ctrl + C_ERR;
  c.s.timeout = p.timeout_ticks;
  c.s.trace = p.trace ? p.trace + (size_t)blockIdx.x * MK_TRACE_SLOTS : nullptr;
  trace_mark(c.s, 0);
  if (LOOP && p.step_clock && blockIdx.x == 0 && tid() == 0) p.step_clock[0] = wall_clock64();
  c.G = GFIX ? GFIX : (int)gridDim.x;
  c.w = blockIdx.x;
  // The control words, the position and the token first; then the first
  // layer's QKV weight ring (it depends on nothing), then the loads that need
  // the position or the token, so that those wait only for the small loads.
  const uint32_t epoch = __hip_atomic_load(ctrl + C_EPOCH, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  c.pos = p.pos[0];
  int tok = p.hidden_in ? 0 : p.tokens[0];
  const int G = c.G, w = c.w, wave = wave_id(), lane = lane_id();
  share(QKV_PAIRS, G, w, c.P0, c.P1);
  c.qkv_n = wave_count(0, 2 * (c.P1 - c.P0));
  RowStream<4, 4> qs;   // the QKV ring of the layer being run
  qkv_ring(c, 0, qs);
  c.set = p.xch + (size_t)(epoch & 1u) * SET_BYTES;
  // refill the other set with the sentinel for the next step: during the
  // lm_head phase of step n, where the stores delay nothing, or here if there
  // is none (step n uses set (epoch + n) & 1)
  auto refill = [&](int step) {
    u32x4* other = reinterpret_cast<u32x4*>(p.xch + (size_t)((epoch + (uint32_t)step + 1u) & 1u) * SET_BYTES);
    const size_t n = SET_BYTES / 16;
    int lo, hi;
    share((int)n, c.G, c.w, lo, hi);
    for (int i = lo + tid(); i < hi; i += NT) other[i] = u32x4{~0u, ~0u, ~0u, ~0u};
  };
  const int pos0 = c.pos;   // a loop's step n runs at position pos0 + n
  const bool pos_ok = c.pos >= 0 && c.pos + n_steps <= p.s_max && c.pos + n_steps <= p.rope_rows;
  if (!p.do_lm || !pos_ok) refill(0);   // (the lm_head phase runs only with a valid position)
  if (!pos_ok && blockIdx.x == 0 && tid() == 0)
    __hip_atomic_fetch_or(c.s.err, MK_DEVERR_POS, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  c.n_rows = c.pos + 1;
  if (p.hidden_in) {
    c.x_in = p.hidden_in;
  } else {
    tok = tok < 0 ? 0 : (tok >= VOCAB ? VOCAB - 1 : tok);
    c.x_in = p.embed + (size_t)tok * H;
  }
  // Decode loop: step n (> 0) starts when every workgroup has finished step
  // n - 1 (arrivals on STEP_LINES sub-counters) and its greedy token is in
  // the argmax key of that step's parity; its layer-0 QKV weights are already
  // in flight, and idle() (the layer-0 gate/up LDS copies) runs between polls.
  auto key_ptr = [&](int n) { return reinterpret_cast<unsigned long long*>(p.ws + C_KEY_BYTE + 64 * (n & 1)); };
  auto step_entry = [&](int n, auto&& idle) {
    const uint32_t per = (uint32_t)(G / STEP_LINES), extra = (uint32_t)(G % STEP_LINES);
    const rsrc_t r = make_rsrc(p.step_cnt, STEP_CNT_BYTES);
    const uint32_t off = lane < STEP_LINES ? (uint32_t)lane * (uint32_t)STEP_LINE : OOB;
    const uint32_t target = lane < STEP_LINES ? (uint32_t)n * (per + ((uint32_t)lane < extra ? 1u : 0u)) : 0u;
    const unsigned long long t0 = wall_clock64();
    for (int it = 1;; ++it) {
      const uint32_t v = ld_dev4(r, off);
      if (__all(v >= target)) break;
      if (wait_expired(c.s, t0, it)) break;
      idle();
      __builtin_amdgcn_s_sleep(1);
    }
    trace_mark(c.s, MK_TRACE_SLOTS - 3);   // (a loop's trace keeps its last step: this step's barrier seen)
    const unsigned long long key = __hip_atomic_load(key_ptr(n - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    trace_mark(c.s, MK_TRACE_SLOTS - 2);
    int t = (int)(0xffffffffu - (uint32_t)(key & 0xffffffffull));
    if (w == 0 && tid() == 0) {
      if (p.tokens_out) p.tokens_out[n - 1] = t;
      if (p.step_clock) p.step_clock[n] = wall_clock64();
    }
    t = t < 0 ? 0 : (t >= VOCAB ? VOCAB - 1 : t);
    c.x_in = p.embed + (size_t)t * H;
  };

  if (pos_ok) for (int n = 0; n < n_steps; ++n) {
    const bool last_step = n + 1 == n_steps;
    if (n > 0) {
      c.pos = pos0 + n;
      c.n_rows = c.pos + 1;
      c.set = p.xch + (size_t)((epoch + (uint32_t)n) & 1u) * SET_BYTES;
    }
    // the step's RoPE row, read once; it goes to LDS with the first layer's input
    uint32_t rope_v = 0;
    if (tid() < HD) rope_v = reinterpret_cast<const uint32_t*>(p.rope + (size_t)c.pos * (2 * HD))[tid()];
    {
      {
        const int ng = (c.n_rows + 31) >> 5;
        c.nsplit = ng < ATT_MAX_SPLIT ? ng : ATT_MAX_SPLIT;
      }
      int R0, R1;
      share(H, G, w, R0, R1);
      c.d_rows = wave_span(R0, R1);
      // O rows: the workgroups that run attention items (and merge the splits)
      // get none, so h1 does not wait for the ones that finish attention last.
      // With eight splits per head, neither do the other workgroups below
      // G - 128 (they start the gate/up prefetch instead): the last 128 take
      // 16 rows each, O_RING per wave, one transposed reduction. (The 192
      // workgroups from 64 on, 10-11 rows each: C3 steps 5 us longer; counts
      // that put more than O_RING rows on a wave: 15-30 us longer.)
      int O0 = R0, O1 = R1;
      const int A = NKV * c.nsplit;   // workgroups [0, A) run attention items
      if (A <= G / 2) {
        // workgroups [0, NO) have no O rows
        const int NO = A == NKV * ATT_MAX_SPLIT ? max(A, G - H / (NWAVE * O_RING)) : A;
        if (w < NO) O0 = O1 = 0;
        else share(H, G - NO, w - NO, O0, O1);
      }
      c.o_rows = wave_span(O0, O1);
      c.has_o = O1 > O0;
      int U0, U1;
      share(INTER, G, w, U0, U1);
      c.gu_pairs = wave_span(U0, U1);
    }
    for (int li = 0; li < p.n_layers; ++li) {
      const int l = p.first_layer + li;
      const bool last = li == p.n_layers - 1;
      // The first GU_LDS_PAIRS gate/up pairs of each wave's GU share go HBM -> LDS
      // directly while the layer waits for its input and its attention output,
      // a few chunks per poll round: the hand-over polls queue behind them
      // (vector loads complete in order), so the copy is spread out.
      GuPrefetch gpf;
      gpf.start(p.w_gu + (size_t)l * 2 * INTER * H, c.gu_pairs, L.gu[__builtin_amdgcn_readfirstlane(wave)]);
      auto gidle = [&]() { gpf.issue_fixed<GU_LDS_STEP_QKV>(L.spare); };
      auto oidle = [&]() { gpf.issue_fixed<GU_LDS_STEP_O>(L.spare); };
      if (li > 0) qkv_ring(c, li, qs);
      if constexpr (LOOP) {
        if (li == 0 && n > 0) step_entry(n, gidle);
      }
      phase_qkv(c, li, L, gidle, qs, [&]() {
        if (li == 0 && tid() < HD) reinterpret_cast<uint32_t*>(L.rope)[tid()] = rope_v;
      });
      if (li == 8) trace_value(c.s, 1, (unsigned long long)gpf.next);
      phase_attn(c, li, L);

      // ---- O projection + residual -> h1 ----
      const uint16_t* w_gu_l = p.w_gu + (size_t)l * 2 * INTER * H;
      GuEarly ge;
      if (!c.has_o) {
        gpf.issue(GU_LDS_PAIRS * 8);
        ge.issue(w_gu_l, c.gu_pairs, gpf.total / 8);
      } else {
        RowStream<O_RING, 4> os;
        const Span sp = c.o_rows;
        os.start(make_rsrc(p.w_o + (size_t)l * H * H, O_LAYER_BYTES), (uint32_t)sp.lo * (H * 2), H * 2, sp.n);
        ge.issue(w_gu_l, c.gu_pairs, gpf.total / 8);
        trace_mark(c.s, 2 * xk(li, 3) - 1);
        stage_vec<1>(c.s, c.xb(li, X_ATT), true, L.v, oidle);
        if (li == 8) trace_value(c.s, 0, (unsigned long long)gpf.next);
        gpf.issue(GU_LDS_PAIRS * 8);   // whatever the waits left
        lds_sync();
        trace_mark(c.s, 2 * xk(li, 3));
        u32x4 xs[4];
        lds_x2048(L.v, xs);
        uint16_t* h1 = c.xb(li, X_H1);
        auto dotf = [&](const u32x4(&wv)[4]) { return dot2048(wv, xs); };
        if (sp.n <= O_RING) {   // one transposed reduction: row r in lanes 16r .. 16r+15
          float pt[O_RING];
          os.dots(dotf, pt);
          const float v = reduce_rows<O_RING>(pt);
          const int r = lane / (64 / O_RING);
          if ((lane & (64 / O_RING - 1)) == 0 && r < sp.n)
            st_dev(h1 + sp.lo + r, f2bf(bf2f(L.x[sp.lo + r]) + rbf(v)));
        } else {
          float mine = 0.f;   // lane r: the wave's row r
          os.run(dotf, [&](int r, float part) {
            const float v = wave_sum(part);
            if (lane == r) mine = v;
          });
          if (lane < sp.n) st_dev(h1 + sp.lo + lane, f2bf(bf2f(L.x[sp.lo + lane]) + rbf(mine)));
        }
        trace_done(c.s, li, 2);
      }

      // ---- gate/up + SwiGLU -> act ----
      const rsrc_t rd = make_rsrc(p.w_d + (size_t)l * H * INTER, D_LAYER_BYTES);
      const bool d_fast = c.d_rows.n <= 2;
      u32x4 dpre[D_EARLY > 0 ? D_EARLY : 1];
      {
        RowStream<GU_RING, 8> gs;
        const Span sp = c.gu_pairs;
        const int n_lds = gpf.total / 8;   // pairs [0, n_lds) are in LDS, the next GU_EARLY in ge
        const int n_reg = min(GU_EARLY, sp.n - n_lds);
        gs.start(make_rsrc(w_gu_l, GU_LAYER_BYTES), (uint32_t)(sp.lo + n_lds + n_reg) * (2 * H * 2), 2 * H * 2,
                 sp.n - n_lds - n_reg);
        trace_mark(c.s, 2 * xk(li, 4) - 1);
        stage_vec<1>(c.s, c.xb(li, X_H1), true, L.h1);
        lds_sync();
        trace_mark(c.s, 2 * xk(li, 4));
        u32x4 xs[4];
        lds_x2048(L.h1, xs);
        rmsnorm2048(xs, nullptr);
        uint16_t* act = c.xb(li, X_ACT);
        struct GU2 { float g, u; };
        float mine = 0.f;   // lane r: silu(gate) * up of the wave's pair r
        auto gu_dot = [&](const u32x4(&wv)[8]) {
          float g0 = dot8(wv[0], xs[0], 0.f), g1 = dot8(wv[1], xs[1], 0.f);
          float u0 = dot8(wv[4], xs[0], 0.f), u1 = dot8(wv[5], xs[1], 0.f);
          g0 = dot8(wv[2], xs[2], g0);
          g1 = dot8(wv[3], xs[3], g1);
          u0 = dot8(wv[6], xs[2], u0);
          u1 = dot8(wv[7], xs[3], u1);
          return GU2{g0 + g1, u0 + u1};
        };
        auto gu_emit = [&](int r, GU2 part) {
          const float gv = wave_sum(part.g);
          const float uv = wave_sum(part.u);
          if (lane == r) mine = gv / (1.0f + __expf(-gv)) * uv;
        };
        wait_mem();   // this wave's LDS copy (and the ring) have landed
        // the first D_EARLY chunks of the wave's first down row (fast down path only)
        {
          const uint32_t o =
              (d_fast && c.d_rows.n > 0 ? (uint32_t)c.d_rows.lo * (INTER * 2) : OOB) + (uint32_t)lane * 16u;
#pragma unroll
          for (int i = 0; i < D_EARLY; ++i) dpre[i] = ld_stream(rd, o + (uint32_t)i * 1024u);
        }
        const uint8_t* src = L.gu[wave];
        auto lds_pair = [&](int j, u32x4(&wv)[8]) {
#pragma unroll
          for (int i = 0; i < 8; ++i) wv[i] = *reinterpret_cast<const u32x4*>(src + (j * 8 + i) * 1024 + lane * 16);
        };
        if (n_lds == GU_LDS_PAIRS && sp.n - n_lds <= 4) {
          // 8 pairs: 16 rows (g of pairs 0-7, then u) in one transposed reduction
          float pt[16];
#pragma unroll
          for (int j = 0; j < GU_LDS_PAIRS; ++j) {
            u32x4 wv[8];
            lds_pair(j, wv);
            const GU2 d = gu_dot(wv);
            pt[j] = d.g;
            pt[8 + j] = d.u;
          }
#pragma unroll
          for (int j = 0; j < GU_EARLY; ++j) {
            const GU2 d = gu_dot(ge.buf[j]);
            pt[GU_LDS_PAIRS + j] = d.g;
            pt[8 + GU_LDS_PAIRS + j] = d.u;
          }
          GU2 rp[GU_RING];
          gs.dots(gu_dot, rp);
#pragma unroll
          for (int j = 0; j < GU_RING; ++j) {
            pt[GU_LDS_PAIRS + GU_EARLY + j] = rp[j].g;
            pt[8 + GU_LDS_PAIRS + GU_EARLY + j] = rp[j].u;
          }

          const float v = reduce_rows<16>(pt);   // lane 4k..4k+3: row k
          const Pair gu = xor32_pair(v);         // lanes 0-31: g (own) and u (lane + 32)
          const int r = lane >> 2;
          if (lane < 32 && (lane & 3) == 0 && r < sp.n) st_dev(act + sp.lo + r, f2bf(gu.a / (1.0f + __expf(-gu.a)) * gu.b));
        } else {
          for (int j = 0; j < n_lds; ++j) {
            u32x4 wv[8];
            lds_pair(j, wv);
            gu_emit(j, gu_dot(wv));
          }
#pragma unroll
          for (int j = 0; j < GU_EARLY; ++j)
            if (j < n_reg) gu_emit(n_lds + j, gu_dot(ge.buf[j]));
          gs.run(gu_dot, [&](int r, GU2 part) { gu_emit(n_lds + n_reg + r, part); });
          if (lane < sp.n) st_dev(act + sp.lo + lane, f2bf(mine));
        }
        trace_done(c.s, li, 3);
      }

      // ---- down projection + residual -> h2 ----
      {
        RowStream<2, 16> ds;
        const Span sp = c.d_rows;
        ds.start(rd, (uint32_t)sp.lo * (INTER * 2), INTER * 2, sp.n, d_fast ? D_EARLY : 0);
        trace_mark(c.s, 2 * xk(li, 5) - 1);
        stage_vec<4>(c.s, c.xb(li, X_ACT), true, L.v);
        lds_sync();
        trace_mark(c.s, 2 * xk(li, 5));

        uint16_t* h2 = c.xb(li, X_H2);
        u32x4 xs[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) xs[i] = *reinterpret_cast<const u32x4*>(L.v + i * 512 + lane * 8);
        auto dotf = [&](const u32x4(&wv)[16]) {
          float a = 0.f, b = 0.f;
#pragma unroll
          for (int i = 0; i < 16; i += 2) {
            a = dot8(wv[i], xs[i], a);
            b = dot8(wv[i + 1], xs[i + 1], b);
          }
          return a + b;
        };
        auto out = [&](int r, float v) {
          const int row = sp.lo + r;
          const uint32_t hv = f2bf(bf2f(L.h1[row]) + rbf(v));
          st_dev(h2 + row, hv);
          if (last && last_step && p.hidden_out) p.hidden_out[row] = (uint16_t)hv;
        };
        if (sp.n <= 2) {   // lanes 0-31: row 0, lanes 32-63: row 1
          float pt[2];
          ds.dots(dotf, pt);
          {   // row 0's first D_EARLY chunks (read as zero by the ring)
            float a = 0.f;
#pragma unroll
            for (int i = 0; i < D_EARLY; ++i) a = dot8(dpre[i], xs[i], a);
            pt[0] += a;
          }
          const float v = reduce_rows<2>(pt);
          const int r = lane >> 5;
          if ((lane & 31) == 0 && r < sp.n) out(r, v);
        } else {
          float mine = 0.f;   // lane r: the wave's row r
          ds.run(dotf, [&](int r, float part) {
            const float v = wave_sum(part);
            if (lane == r) mine = v;
          });
          if (lane < sp.n) out(lane, mine);
        }
        trace_done(c.s, li, 4);
      }
    }

    // ---- final norm + tied lm_head + argmax ----
    if (p.do_lm) {
      int V0, V1;
      share(VOCAB, G, w, V0, V1);
      RowStream<LM_RING, 4> ls;
      const Span sp = wave_span(V0, V1);
      ls.start(make_rsrc(p.embed, EMBED_BYTES), (uint32_t)sp.lo * (H * 2), H * 2, sp.n);
      trace_mark(c.s, 2 * xk(p.n_layers, 1) - 1);
      stage_vec<1>(c.s, c.xb(p.n_layers - 1, X_H2), true, L.x);
      lds_sync();
      trace_mark(c.s, 2 * xk(p.n_layers, 1));
      refill(n);
      // the next step's argmax key (read by every workgroup at the start of
      // this step, all of which have passed their first hand-overs by now)
      if (!last_step && w == 0 && tid() == 0)
        __hip_atomic_store(key_ptr(n + 1), 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      u32x4 xs[4];
      lds_x2048(L.x, xs);
      rmsnorm2048(xs, p.g_final);
      float best = -INFINITY;
      int bidx = 0x7fffffff;
      ls.run([&](const u32x4(&wv)[4]) { return dot2048(wv, xs); },
             [&](int r, float part) {
               const float v = wave_sum(part);
               const int row = sp.lo + r;
               if (lane == 0 && p.logits && last_step) p.logits[row] = v;
               if (v > best) {   // rows ascend: keeps the lowest index among equal maxima
                 best = v;
                 bidx = row;
               }
             });
      if (lane == 0) {
        L.best[wave] = best;
        L.bidx[wave] = bidx;
      }
      __syncthreads();
      if (tid() == 0) {
        float b = L.best[0];
        int bi = L.bidx[0];
        for (int k = 1; k < NWAVE; ++k)
          if (L.best[k] > b || (L.best[k] == b && L.bidx[k] < bi)) {
            b = L.best[k];
            bi = L.bidx[k];
          }
        if (bi != 0x7fffffff) {
          uint32_t u = __float_as_uint(b);
          u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);   // order-preserving float key
          const unsigned long long key =
              ((unsigned long long)u << 32) | (unsigned long long)(0xffffffffu - (uint32_t)bi);
          __hip_atomic_fetch_max(key_ptr(n), key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
    if (!last_step) {
      // this workgroup's step is complete (its stores, the K/V rows included,
      // and its argmax contribution): one arrival; then the next step's
      // layer-0 QKV weights go in flight
      wait_mem();
      __syncthreads();
      trace_mark(c.s, MK_TRACE_SLOTS - 4);   // the step's arrival
      if (tid() == 0)
        __hip_atomic_fetch_add(p.step_cnt + (size_t)(w % STEP_LINES) * (STEP_LINE / 4), 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
      qkv_ring(c, 0, qs);
    }
  }

  // ---- exit: the last workgroup out publishes the token and advances the epoch ----
  trace_mark(c.s, MK_TRACE_SLOTS - 1);
  wait_mem();
  __syncthreads();
  if (tid() == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(ctrl + C_EXIT, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    L.last = prev == (uint32_t)(G - 1);
  }
  __syncthreads();
  if (!L.last || tid() != 0) return;
  ctrl[C_EXIT] = 0u;
  ctrl[C_EPOCH] = epoch + (pos_ok ? (uint32_t)n_steps : 1u);
  unsigned long long key = 0ull;
  if (pos_ok && p.do_lm) {
    unsigned long long* kp = key_ptr(n_steps - 1);
    key = __hip_atomic_load(kp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *kp = 0ull;
  }
  if constexpr (LOOP) {
    if (n_steps > 1) {   // both keys and the step counters start the next launch at zero
      *key_ptr(n_steps) = 0ull;
      for (int j = 0; j < STEP_LINES; ++j) p.step_cnt[(size_t)j * (STEP_LINE / 4)] = 0u;
    }
    if (p.step_clock) p.step_clock[n_steps] = wall_clock64();
    if (pos_ok && p.tokens_out) p.tokens_out[n_steps - 1] = (int32_t)(0xffffffffu - (uint32_t)(key & 0xffffffffull));
  }
  if (p.noalloc) {
    // In the static scratch the step's error bits are cleared so the next
    // step's waits do not bail out; a faulted step reports next_token = -1
    // (if given), does not advance, and ORs its bits into the sticky word that
    // mk_read_device_error(NULL, ...) returns and clears.
    const uint32_t bits = __hip_atomic_load(ctrl + C_ERR, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    ctrl[C_ERR] = 0u;
    if (bits) {
      __hip_atomic_fetch_or(ctrl + C_STICKY, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (p.next_token) p.next_token[0] = -1;
      return;
    }
  }
  if (pos_ok) {
    if (p.do_lm && p.next_token) p.next_token[0] = (int32_t)(0xffffffffu - (uint32_t)(key & 0xffffffffull));
    if (p.flags & MK_FLAG_ADVANCE) p.pos[0] = c.pos + 1;
  }
}

// Fill kernel: the first n_zero 16-byte units zeroed (the control block), the
// rest set to the exchange sentinel (all ones).
__global__ void mk_ws_init_kernel(u32x4* p, size_t n, size_t n_zero) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + tid(); i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = i < n_zero ? u32x4{0u, 0u, 0u, 0u} : u32x4{~0u, ~0u, ~0u, ~0u};
}

}  // namespace

#ifdef MK_DECODE_STEP_TU

namespace mk {
// The single-step kernel of this translation unit for a grid of `grid` workgroups.
const void* decode_step_kernel(int grid) {
  return grid == 256 ? reinterpret_cast<const void*>(mk_decode_kernel<256, false>)
                     : reinterpret_cast<const void*>(mk_decode_kernel<0, false>);
}
}  // namespace mk

#else

namespace mk {
const void* decode_step_kernel(int grid);   // mk_decode_step.hip
}  // namespace mk

namespace {

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
thread_local char g_msg[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
  va_end(ap);
  return code;
}

struct DeviceInfo {
  int ready;
  int grid;        // workgroups per launch: the CU count, or the mk_set_grid_size override
  int cus;
  unsigned long long ticks_per_s;
  int status;
};
DeviceInfo g_dev[64];
std::mutex g_dev_mu;

// The batch-1 kernel for a grid of `grid` workgroups (one per CU): MI355X's 256
// CUs get the instantiations with the grid size fixed at compile time; `loop`
// selects the decode loop's instantiation.
const void* decode_kernel_for(int grid, bool loop = false) {
  if (loop)
    return grid == 256 ? reinterpret_cast<const void*>(mk_decode_kernel<256, true>)
                       : reinterpret_cast<const void*>(mk_decode_kernel<0, true>);
  return decode_step_kernel(grid);
}

int device_info(int dev, DeviceInfo* out) {
  if (dev < 0 || dev >= 64) return fail(MK_ERR_DEVICE, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_dev_mu);
  DeviceInfo& d = g_dev[dev];
  if (!d.ready) {
    int cus = 0, coop = 0, clk_khz = 0, nb = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess ||
        hipDeviceGetAttribute(&clk_khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess)
      return fail(MK_ERR_HIP, "hipDeviceGetAttribute failed on device %d", dev);
    d.grid = cus;
    d.cus = cus;
    int nbl = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, decode_kernel_for(cus), NT, 0) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&nbl, decode_kernel_for(cus, true), NT, 0) != hipSuccess)
      return fail(MK_ERR_HIP, "occupancy query failed");
    nb = nb < nbl ? nb : nbl;
    d.ticks_per_s = (unsigned long long)(clk_khz > 0 ? clk_khz : 100000) * 1000ull;
    d.status = MK_OK;
    if (!coop) d.status = fail(MK_ERR_DEVICE, "device %d lacks cooperative launch", dev);
    else if (nb < 1) d.status = fail(MK_ERR_DEVICE, "kernel cannot be resident on a CU (occupancy %d)", nb);
    else if (cus < MIN_GRID || cus > MAX_GRID) d.status = fail(MK_ERR_DEVICE, "unsupported CU count %d", cus);
    d.ready = 1;
  }
  *out = d;
  return d.status;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Exchange areas, one per initialised workspace and device, created by its
// first mk_workspace_init there and kept until the process ends.
//   * batch-1 workspaces: XCH_BYTES of uncached device memory. The per-layer
//     hand-over buffers are polled there: an all-to-all hand-over under a full
//     HBM weight stream took 3.8 us against 6 us in ordinary (L2-cached)
//     memory. Uncached memory that a kernel has read must not be freed while
//     the process runs.
//   * batched workspaces (max batch M >= 2): BatchLayout(M).total bytes of
//     ordinary device memory, whose activation matrices every workgroup reads
//     through its XCD's L2.
//     Its arrival counters sit in a BCNT_BLOCK_BYTES block of uncached memory
//     of the entry (`cnt`): a counter hand-over polled there under a full
//     weight stream completes sooner than one polled in ordinary memory.
// A workspace re-initialised with another layout (a new allocation at the
// same address) gets a matching area; areas it no longer uses stay in the
// list and are handed to the next workspace that fits. mk_workspace_release
// returns a workspace's area: an uncached one becomes spare (never freed), an
// ordinary one is freed and its entry removed, its counter block kept in a
// spare list for the next batched workspace on the device.
constexpr size_t XCH_BYTES = 2 * SET_BYTES;
struct XchEntry {
  const void* ws;   // owner (nullptr: spare)
  int dev;
  int max_batch;    // 1: batch-1 layout
  size_t bytes;
  uint8_t* xch;
  uint8_t* cnt;     // batched: uncached counter block (nullptr for batch-1 entries)
};
XchEntry g_xch[256];
int g_n_xch = 0;
struct CntBlock {
  int dev;
  uint8_t* p;
};
CntBlock g_cnt_spare[256];   // counter blocks of released batched areas (uncached: never freed)
int g_n_cnt_spare = 0;
std::mutex g_xch_mu;

// An uncached counter block for a new batched entry on `dev` (caller holds g_xch_mu).
int counter_block(int dev, uint8_t** out) {
  for (int i = 0; i < g_n_cnt_spare; ++i)
    if (g_cnt_spare[i].dev == dev) {
      *out = g_cnt_spare[i].p;
      g_cnt_spare[i] = g_cnt_spare[--g_n_cnt_spare];
      return MK_OK;
    }
  void* p = nullptr;
  const hipError_t e = hipExtMallocWithFlags(&p, BCNT_BLOCK_BYTES, hipDeviceMallocUncached);
  if (e != hipSuccess) return fail(MK_ERR_HIP, "counter block allocation: %s", hipGetErrorString(e));
  *out = static_cast<uint8_t*>(p);
  return MK_OK;
}

bool exchange_of(const void* ws, int dev, XchEntry* out) {
  std::lock_guard<std::mutex> lk(g_xch_mu);
  for (int i = 0; i < g_n_xch; ++i)
    if (g_xch[i].ws == ws && g_xch[i].dev == dev) {
      *out = g_xch[i];
      return true;
    }
  return false;
}

int exchange_create(const void* ws, int dev, int max_batch, XchEntry* out) {
  const bool uncached = max_batch == 1;
  size_t need = XCH_BYTES + STEP_CNT_BYTES;   // batch 1: the two sets, then the decode loop's step counters
  if (!uncached) {
    BatchLayout lay;
    lay.init(max_batch);
    need = lay.total;
  }
  std::lock_guard<std::mutex> lk(g_xch_mu);
  int mine = -1;
  for (int i = 0; i < g_n_xch; ++i)
    if (g_xch[i].ws == ws && g_xch[i].dev == dev) mine = i;
  if (mine >= 0) {
    XchEntry& e = g_xch[mine];
    if ((e.max_batch == 1) == uncached && e.bytes >= need) {
      e.max_batch = max_batch;
      *out = e;
      return MK_OK;
    }
    e.ws = nullptr;   // spare
  }
  for (int i = 0; i < g_n_xch; ++i) {
    XchEntry& e = g_xch[i];
    if (e.ws == nullptr && e.dev == dev && (e.max_batch == 1) == uncached && e.bytes >= need) {
      e.ws = ws;
      e.max_batch = max_batch;
      *out = e;
      return MK_OK;
    }
  }
  if (g_n_xch == (int)(sizeof(g_xch) / sizeof(g_xch[0])))
    return fail(MK_ERR_WORKSPACE, "too many workspaces initialised in this process (%d)", g_n_xch);
  uint8_t* cnt = nullptr;
  if (!uncached) {
    const int rc = counter_block(dev, &cnt);
    if (rc != MK_OK) return rc;
  }
  void* p = nullptr;
  const hipError_t e = uncached ? hipExtMallocWithFlags(&p, need, hipDeviceMallocUncached) : hipMalloc(&p, need);
  if (e != hipSuccess) {
    if (cnt) g_cnt_spare[g_n_cnt_spare++] = CntBlock{dev, cnt};
    return fail(MK_ERR_HIP, "exchange area allocation (%zu bytes): %s", need, hipGetErrorString(e));
  }
  g_xch[g_n_xch++] = XchEntry{ws, dev, max_batch, need, static_cast<uint8_t*>(p), cnt};
  *out = g_xch[g_n_xch - 1];
  return MK_OK;
}

// Release the exchange area owned by `ws` on `dev` (see above). The caller
// has synchronised the device, so no kernel still uses the area.
int exchange_release(const void* ws, int dev) {
  std::lock_guard<std::mutex> lk(g_xch_mu);
  for (int i = 0; i < g_n_xch; ++i) {
    XchEntry& e = g_xch[i];
    if (e.ws != ws || e.dev != dev) continue;
    if (e.max_batch == 1) {   // uncached: read by kernels, so kept until the process ends
      e.ws = nullptr;
      return MK_OK;
    }
    const hipError_t he = hipFree(e.xch);
    g_cnt_spare[g_n_cnt_spare++] = CntBlock{dev, e.cnt};
    g_xch[i] = g_xch[--g_n_xch];
    if (he != hipSuccess) return fail(MK_ERR_HIP, "freeing the exchange area: %s", hipGetErrorString(he));
    return MK_OK;
  }
  return fail(MK_ERR_WORKSPACE, "workspace %p has no exchange area on device %d", ws, dev);
}


// Argument checks shared by mk_decode_step and mk_decode_step_noalloc (all but the workspace).
int check_step_args(const mk_weights* w, const mk_step_args* a) {
  if (!w || !a) return fail(MK_ERR_NULL, "weights or args is NULL");
  if (a->n_layers < 1 || a->first_layer < 0 || a->first_layer + a->n_layers > w->n_layers ||
      w->n_layers > MK_MAX_LAYERS)
    return fail(MK_ERR_SHAPE, "layers [%d, %d) not within the %d packed layers (max %d)", a->first_layer,
                a->first_layer + a->n_layers, w->n_layers, MK_MAX_LAYERS);
  if (a->batch < 1) return fail(MK_ERR_SHAPE, "batch %d < 1", a->batch);
  if (a->batch > BATCH_MAX) return fail(MK_ERR_SHAPE, "batch %d > %d", a->batch, BATCH_MAX);
  if (a->s_max < 1 || a->s_max > w->rope_rows)
    return fail(MK_ERR_SHAPE, "s_max %d must be in [1, rope_rows=%d]", a->s_max, w->rope_rows);
  if (!a->k_cache || !a->v_cache) return fail(MK_ERR_NULL, "k_cache / v_cache array is NULL");
  for (int i = 0; i < a->n_layers; ++i) {
    if (!a->k_cache[i] || !a->v_cache[i]) return fail(MK_ERR_NULL, "cache pointer of layer %d is NULL", i);
    if (!aligned16(a->k_cache[i]) || !aligned16(a->v_cache[i]))
      return fail(MK_ERR_ALIGN, "cache of layer %d is not 16-byte aligned", i);
  }
  if ((a->tokens == nullptr) == (a->hidden_in == nullptr))
    return fail(MK_ERR_NULL, "exactly one of tokens / hidden_in must be given");
  if (!a->pos) return fail(MK_ERR_NULL, "pos is NULL");
  const bool do_lm = a->logits != nullptr || a->next_token != nullptr;
  if (!w->w_qkv || !w->w_o || !w->w_gu || !w->w_down || !w->rope)
    return fail(MK_ERR_NULL, "a layer weight pointer is NULL");
  if ((do_lm || a->tokens) && !w->embed) return fail(MK_ERR_NULL, "embed is NULL");
  if (do_lm && !w->norm_final) return fail(MK_ERR_NULL, "norm_final is NULL");
  const void* al[] = {w->w_qkv, w->w_o, w->w_gu, w->w_down, w->embed, w->norm_final, a->hidden_in, a->hidden_out};
  for (const void* q : al)
    if (q && !aligned16(q)) return fail(MK_ERR_ALIGN, "a weight or hidden pointer is not 16-byte aligned");
  return MK_OK;
}

// Enqueue mk_decode_kernel (batch 1) with control block `ctrl` and exchange sets `xch`.
int launch_decode(const mk_weights* w, const mk_step_args* a, const DeviceInfo& di, uint8_t* ctrl, uint8_t* xch,
                  bool noalloc, int n_steps = 1, int32_t* tokens_out = nullptr, uint64_t* step_clock = nullptr) {
  // (a loop, or a caller of it that asks for the tokens, needs every step's argmax)
  const bool do_lm = a->logits != nullptr || a->next_token != nullptr || n_steps > 1 || tokens_out != nullptr;
  KParams kp;
  memset(&kp, 0, sizeof(kp));
  kp.w_qkv = static_cast<const uint16_t*>(w->w_qkv);
  kp.w_o = static_cast<const uint16_t*>(w->w_o);
  kp.w_gu = static_cast<const uint16_t*>(w->w_gu);
  kp.w_d = static_cast<const uint16_t*>(w->w_down);
  kp.embed = static_cast<const uint16_t*>(w->embed);
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
  kp.ws = ctrl;
  kp.xch = xch;
  kp.first_layer = a->first_layer;
  kp.n_layers = a->n_layers;
  kp.s_max = a->s_max;
  kp.rope_rows = w->rope_rows;
  kp.do_lm = do_lm ? 1 : 0;
  kp.noalloc = noalloc ? 1 : 0;
  kp.flags = a->flags;
  kp.timeout_ticks = di.ticks_per_s * 2ull;   // 2 s per hand-over wait
  kp.trace = static_cast<unsigned long long*>(a->trace);
  kp.n_steps = n_steps;
  kp.tokens_out = tokens_out;
  kp.step_clock = reinterpret_cast<unsigned long long*>(step_clock);
  kp.step_cnt = n_steps > 1 ? reinterpret_cast<uint32_t*>(xch + XCH_BYTES) : nullptr;

  void* args[] = {&kp};
  // One workgroup per CU with occupancy 1 (checked in device_info): on an
  // otherwise idle device a plain launch makes every workgroup resident at
  // once, and leaves ~20 us less between consecutive steps than a cooperative
  // launch. MK_FLAG_COOPERATIVE asks for the guarantee. Every wait in the
  // kernel is bounded, so a workgroup that is never scheduled shows up as
  // MK_DEVERR_SYNC, not as a hang.
  const hipStream_t st = static_cast<hipStream_t>(a->stream);
  const void* fn = decode_kernel_for(di.grid, n_steps > 1 || tokens_out || step_clock);
  const hipError_t e = (a->flags & MK_FLAG_COOPERATIVE)
                           ? hipLaunchCooperativeKernel(fn, dim3(di.grid), dim3(NT), args, 0, st)
                           : hipLaunchKernel(fn, dim3(di.grid), dim3(NT), args, 0, st);
  if (e != hipSuccess) return fail(MK_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e));
  return MK_OK;
}

// Scratch of mk_decode_step_noalloc, for callers that cannot allocate: the
// batch-1 control block followed by both exchange sets, in ordinary device
// memory (each device that runs the library holds its own copy until the
// process ends). Host code never uses the array's name as an address (on the
// host it is only a stand-in for the symbol): the device address comes from
// hipGetSymbolAddress, once per device.
constexpr size_t NOALLOC_SCRATCH_BYTES = CTRL_BYTES + XCH_BYTES;   // 3,277,056 bytes
static_assert(NOALLOC_SCRATCH_BYTES == 3277056, "scratch size stated in mk.h");
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

struct NoAllocDev {
  uint8_t* ptr;    // device address of `scratch` on this device
  bool filled;     // its initial fill has run outside stream capture
};
NoAllocDev g_noalloc[64];
std::mutex g_noalloc_mu;

// The device's scratch address (looked up on its first use there, with the
// device current); until a fill has run outside stream capture, a fill kernel
// (control block zero, exchange sets the sentinel) is enqueued first on `st`.
int noalloc_scratch(int dev, hipStream_t st, uint8_t** out) {
  if (dev < 0 || dev >= 64) return fail(MK_ERR_DEVICE, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  NoAllocDev& d = g_noalloc[dev];
  if (!d.ptr) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(MK_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    d.ptr = static_cast<uint8_t*>(ptr);
  }
  if (!d.filled) {
    hipLaunchKernelGGL(mk_ws_init_kernel, dim3(1024), dim3(256), 0, st, reinterpret_cast<u32x4*>(d.ptr),
                       NOALLOC_SCRATCH_BYTES / 16, CTRL_BYTES / 16);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(MK_ERR_HIP, "scratch fill launch: %s", hipGetErrorString(e));
    // A fill recorded into a graph under capture has not run yet: fill again
    // on the next call outside capture.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusActive;
    if (hipStreamIsCapturing(st, &cs) == hipSuccess && cs == hipStreamCaptureStatusNone) d.filled = true;
  }
  *out = d.ptr;
  return MK_OK;
}

}  // namespace

extern "C" {

int mk_abi_version(void) { return MK_ABI_VERSION; }

const char* mk_last_error(void) { return g_msg; }

int mk_grid_size(int device) {
  DeviceInfo d;
  const int rc = device_info(device, &d);
  return rc == MK_OK ? d.grid : rc;
}

int mk_set_grid_size(int device, int workgroups) {
  DeviceInfo d;
  const int rc = device_info(device, &d);
  if (rc != MK_OK) return rc;
  if (workgroups != 0 && (workgroups < MIN_GRID || workgroups > d.cus))
    return fail(MK_ERR_SHAPE, "grid of %d workgroups not in [%d, %d] (the CU count) on device %d", workgroups,
                MIN_GRID, d.cus, device);
  std::lock_guard<std::mutex> lk(g_dev_mu);
  g_dev[device].grid = workgroups ? workgroups : g_dev[device].cus;
  return MK_OK;
}

long long mk_wall_clock_hz(int device) {
  DeviceInfo d;
  const int rc = device_info(device, &d);
  return rc == MK_OK ? (long long)d.ticks_per_s : rc;
}

size_t mk_workspace_bytes(int32_t batch, int32_t s_max) {
  if (batch < 1 || batch > BATCH_MAX || s_max < 1 || s_max > (1 << 20)) return 0;
  return batch == 1 ? WS_BYTES : batch_ws_bytes(batch);
}

int mk_workspace_init(void* workspace, size_t workspace_bytes, void* stream) {
  if (!workspace) return fail(MK_ERR_NULL, "workspace is NULL");
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) || (workspace_bytes & 15u))
    return fail(MK_ERR_WORKSPACE, "workspace must be 256-byte aligned with a size multiple of 16");
  if (workspace_bytes < WS_BYTES)
    return fail(MK_ERR_WORKSPACE, "workspace %zu bytes < %zu needed", workspace_bytes, WS_BYTES);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(MK_ERR_HIP, "hipGetDevice failed");
  XchEntry xe;
  int rc = exchange_create(workspace, dev, batch_of_ws_bytes(workspace_bytes), &xe);
  if (rc != MK_OK) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t n = workspace_bytes / 16;
  hipLaunchKernelGGL(mk_ws_init_kernel, dim3((int)((n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024)), dim3(256), 0,
                     st, static_cast<u32x4*>(workspace), n, n);
  if (xe.max_batch == 1) {   // batch-1 exchange sets start filled with the sentinel
    hipLaunchKernelGGL(mk_ws_init_kernel, dim3(1024), dim3(256), 0, st, reinterpret_cast<u32x4*>(xe.xch),
                       XCH_BYTES / 16, (size_t)0);
    hipLaunchKernelGGL(mk_ws_init_kernel, dim3(1), dim3(256), 0, st, reinterpret_cast<u32x4*>(xe.xch + XCH_BYTES),
                       STEP_CNT_BYTES / 16, STEP_CNT_BYTES / 16);   // the step counters start at zero
  } else {                   // so do the two sentinel sets of a batched exchange area
    BatchLayout lay;
    lay.init(xe.max_batch);
    hipLaunchKernelGGL(mk_ws_init_kernel, dim3(1024), dim3(256), 0, st,
                       reinterpret_cast<u32x4*>(xe.xch + lay.sent_base), 2 * lay.sset / 16, (size_t)0);
    hipLaunchKernelGGL(mk_ws_init_kernel, dim3(64), dim3(256), 0, st, reinterpret_cast<u32x4*>(xe.cnt),
                       BCNT_BLOCK_BYTES / 16, BCNT_BLOCK_BYTES / 16);   // counters start at zero
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MK_ERR_HIP, "workspace init launch: %s", hipGetErrorString(e));
  return MK_OK;
}

int mk_workspace_release(void* workspace) {
  if (!workspace) return fail(MK_ERR_NULL, "workspace is NULL");
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(MK_ERR_HIP, "hipGetDevice failed");
  // every kernel that may still use the workspace's exchange area has finished
  const hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return fail(MK_ERR_HIP, "hipDeviceSynchronize: %s", hipGetErrorString(e));
  return exchange_release(workspace, dev);
}

int mk_read_device_error(void* workspace, void* stream, uint32_t* bits_out) {
  if (!bits_out) return fail(MK_ERR_NULL, "bits_out is NULL");
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e = hipStreamSynchronize(st);
  if (e != hipSuccess) return fail(MK_ERR_HIP, "hipStreamSynchronize: %s", hipGetErrorString(e));
  uint32_t* dev_err = nullptr;
  if (workspace) {
    dev_err = reinterpret_cast<uint32_t*>(workspace) + C_ERR;
  } else {
    // the allocation-free scratch of the current device (its address from
    // hipGetSymbolAddress; nothing to read before its first use)
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(MK_ERR_HIP, "hipGetDevice failed");
    if (dev < 0 || dev >= 64) return fail(MK_ERR_DEVICE, "device index %d out of range", dev);
    uint8_t* base = nullptr;
    {
      std::lock_guard<std::mutex> lk(g_noalloc_mu);
      base = g_noalloc[dev].ptr;
    }
    if (!base) {
      *bits_out = 0u;
      return MK_OK;
    }
    dev_err = reinterpret_cast<uint32_t*>(base) + C_STICKY;
  }
  uint32_t bits = 0, zero = 0;
  e = hipMemcpy(&bits, dev_err, 4, hipMemcpyDeviceToHost);
  if (e == hipSuccess) e = hipMemcpy(dev_err, &zero, 4, hipMemcpyHostToDevice);
  if (e != hipSuccess) return fail(MK_ERR_HIP, "reading device error: %s", hipGetErrorString(e));
  *bits_out = bits;
  return MK_OK;
}

int mk_decode_step(const mk_weights* w, const mk_step_args* a) {
  int rc = check_step_args(w, a);
  if (rc != MK_OK) return rc;
  if (!a->workspace) return fail(MK_ERR_NULL, "workspace is NULL");
  if (reinterpret_cast<uintptr_t>(a->workspace) & 255u) return fail(MK_ERR_WORKSPACE, "workspace not 256-byte aligned");
  const size_t need = mk_workspace_bytes(a->batch, a->s_max);
  if (a->workspace_bytes < need)
    return fail(MK_ERR_WORKSPACE, "workspace %zu bytes < %zu needed", a->workspace_bytes, need);

  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(MK_ERR_HIP, "hipGetDevice failed");
  DeviceInfo di;
  rc = device_info(dev, &di);
  if (rc != MK_OK) return rc;
  XchEntry xe;
  if (!exchange_of(a->workspace, dev, &xe))
    return fail(MK_ERR_WORKSPACE, "workspace was not initialised with mk_workspace_init on device %d", dev);
  if (a->batch > xe.max_batch)
    return fail(MK_ERR_WORKSPACE, "batch %d exceeds the workspace's batch %d (mk_workspace_bytes)", a->batch,
                xe.max_batch);
  if ((a->flags & MK_FLAG_PREFILL) && xe.max_batch == 1)
    return fail(MK_ERR_UNSUPPORTED, "MK_FLAG_PREFILL needs a batched workspace (mk_workspace_bytes with batch >= 2)");
  if (xe.max_batch > 1) {
    // batched layout: MFMA kernel (mk_batch.hip) for every batch size on this workspace
    if (a->workspace_bytes < batch_ws_bytes(xe.max_batch))
      return fail(MK_ERR_WORKSPACE, "workspace %zu bytes < %zu it was initialised with", a->workspace_bytes,
                  batch_ws_bytes(xe.max_batch));
    const int brc = batch_device_check(dev, g_msg, sizeof(g_msg));
    if (brc != MK_OK) return brc;
    const hipError_t be = batch_launch(w, a, xe.xch, xe.cnt, xe.max_batch, di.grid, di.ticks_per_s * 2ull);
    if (be != hipSuccess) return fail(MK_ERR_HIP, "batched kernel launch failed: %s", hipGetErrorString(be));
    return MK_OK;
  }
  return launch_decode(w, a, di, static_cast<uint8_t*>(a->workspace), xe.xch, false);
}

int mk_decode_loop(const mk_weights* w, const mk_step_args* a, int32_t n_steps, int32_t* tokens_out,
                   uint64_t* step_clock) {
  int rc = check_step_args(w, a);
  if (rc != MK_OK) return rc;
  if (n_steps < 1 || n_steps > (1 << 20)) return fail(MK_ERR_SHAPE, "n_steps %d not in [1, 2^20]", n_steps);
  if (a->batch != 1) return fail(MK_ERR_UNSUPPORTED, "the decode loop runs batch 1 (batch %d)", a->batch);
  if (!a->tokens || a->hidden_in)
    return fail(MK_ERR_UNSUPPORTED, "the decode loop takes token input (each step's token is the last one's argmax)");
  if (!w->norm_final) return fail(MK_ERR_NULL, "norm_final is NULL (every step of the loop runs the lm_head)");
  if (a->flags & MK_FLAG_PREFILL) return fail(MK_ERR_UNSUPPORTED, "MK_FLAG_PREFILL is not a decode loop");
  if ((tokens_out && !aligned16(tokens_out)) || (step_clock && !aligned16(step_clock)))
    return fail(MK_ERR_ALIGN, "tokens_out / step_clock not 16-byte aligned");
  if (!a->workspace) return fail(MK_ERR_NULL, "workspace is NULL");
  if (reinterpret_cast<uintptr_t>(a->workspace) & 255u) return fail(MK_ERR_WORKSPACE, "workspace not 256-byte aligned");
  if (a->workspace_bytes < mk_workspace_bytes(1, a->s_max))
    return fail(MK_ERR_WORKSPACE, "workspace %zu bytes < %zu needed", a->workspace_bytes, mk_workspace_bytes(1, a->s_max));
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(MK_ERR_HIP, "hipGetDevice failed");
  DeviceInfo di;
  rc = device_info(dev, &di);
  if (rc != MK_OK) return rc;
  XchEntry xe;
  if (!exchange_of(a->workspace, dev, &xe))
    return fail(MK_ERR_WORKSPACE, "workspace was not initialised with mk_workspace_init on device %d", dev);
  if (xe.max_batch != 1) return fail(MK_ERR_UNSUPPORTED, "the decode loop needs a batch-1 workspace");
  return launch_decode(w, a, di, static_cast<uint8_t*>(a->workspace), xe.xch, false, n_steps, tokens_out, step_clock);
}

int mk_decode_step_noalloc(const mk_weights* w, const mk_step_args* a) {
  int rc = check_step_args(w, a);
  if (rc != MK_OK) return rc;
  if (a->batch != 1)
    return fail(MK_ERR_SHAPE, "batch %d: the allocation-free step serves batch 1 (its %zu-byte scratch holds the "
                "batch-1 exchange sets)", a->batch, NOALLOC_SCRATCH_BYTES);
  if (a->flags & MK_FLAG_PREFILL)
    return fail(MK_ERR_UNSUPPORTED, "MK_FLAG_PREFILL needs the batched kernel; the allocation-free step is batch 1");
  if (a->workspace || a->workspace_bytes)
    return fail(MK_ERR_WORKSPACE, "the allocation-free step takes no workspace (it uses the library's scratch)");
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(MK_ERR_HIP, "hipGetDevice failed");
  DeviceInfo di;
  rc = device_info(dev, &di);
  if (rc != MK_OK) return rc;
  uint8_t* base = nullptr;
  rc = noalloc_scratch(dev, static_cast<hipStream_t>(a->stream), &base);
  if (rc != MK_OK) return rc;
  return launch_decode(w, a, di, base, base + CTRL_BYTES, true);
}

size_t mk_prefill_workspace_bytes(int32_t chunk_tokens) {
  if (chunk_tokens < 1 || chunk_tokens > PREFILL_MAX_CHUNK) return 0;
  return prefill_ws_bytes(chunk_tokens);
}

int mk_prefill(const mk_weights* w, const mk_prefill_args* a) {
  if (!w || !a) return fail(MK_ERR_NULL, "weights or args is NULL");
  if (a->n_layers < 1 || a->first_layer < 0 || a->first_layer + a->n_layers > w->n_layers ||
      w->n_layers > MK_MAX_LAYERS)
    return fail(MK_ERR_SHAPE, "layers [%d, %d) not within the %d packed layers (max %d)", a->first_layer,
                a->first_layer + a->n_layers, w->n_layers, MK_MAX_LAYERS);
  if (a->n_tokens < 1) return fail(MK_ERR_SHAPE, "n_tokens %d < 1", a->n_tokens);
  if (a->start_pos < 0 || a->s_max < 1 || (long long)a->start_pos + a->n_tokens > a->s_max ||
      a->s_max > w->rope_rows)
    return fail(MK_ERR_SHAPE, "positions [%d, %d) must lie in [0, s_max=%d], s_max <= rope_rows=%d", a->start_pos,
                a->start_pos + a->n_tokens, a->s_max, w->rope_rows);
  if (!a->tokens || !a->k_cache || !a->v_cache) return fail(MK_ERR_NULL, "tokens / k_cache / v_cache is NULL");
  if (!w->w_qkv || !w->w_o || !w->w_gu || !w->w_down || !w->embed || !w->rope)
    return fail(MK_ERR_NULL, "a weight pointer is NULL");
  for (int i = 0; i < a->n_layers; ++i) {
    if (!a->k_cache[i] || !a->v_cache[i]) return fail(MK_ERR_NULL, "cache pointer of layer %d is NULL", i);
    if (!aligned16(a->k_cache[i]) || !aligned16(a->v_cache[i]))
      return fail(MK_ERR_ALIGN, "cache of layer %d not 16-byte aligned", i);
  }
  if (!aligned16(a->tokens) || (a->hidden_out && !aligned16(a->hidden_out)))
    return fail(MK_ERR_ALIGN, "tokens / hidden_out not 16-byte aligned");
  if (!a->workspace) return fail(MK_ERR_NULL, "workspace is NULL");
  if (reinterpret_cast<uintptr_t>(a->workspace) & 255u) return fail(MK_ERR_WORKSPACE, "workspace not 256-byte aligned");
  const int cap = prefill_chunk_cap(a->workspace_bytes);
  if (cap < 1)
    return fail(MK_ERR_WORKSPACE, "workspace %zu bytes < %zu (mk_prefill_workspace_bytes(16))", a->workspace_bytes,
                prefill_ws_bytes(16));
  const hipError_t e = prefill_launch(w, a, cap);
  if (e != hipSuccess) return fail(MK_ERR_HIP, "prefill launch failed: %s", hipGetErrorString(e));
  return MK_OK;
}

int mk_layer_step(const mk_weights* w, int32_t layer, int32_t batch, int32_t s_max, void* k_cache, void* v_cache,
                  const void* hidden_in, int32_t* pos, void* hidden_out, void* workspace, size_t workspace_bytes,
                  void* stream) {
  if (!hidden_in || !hidden_out) return fail(MK_ERR_NULL, "hidden_in / hidden_out is NULL");
  void* kc[1] = {k_cache};
  void* vc[1] = {v_cache};
  mk_step_args a;
  memset(&a, 0, sizeof(a));
  a.first_layer = layer;
  a.n_layers = 1;
  a.batch = batch;
  a.s_max = s_max;
  a.k_cache = kc;
  a.v_cache = vc;
  a.hidden_in = hidden_in;
  a.pos = pos;
  a.hidden_out = hidden_out;
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  a.stream = stream;
  return mk_decode_step(w, &a);
}

}  // extern "C"

#endif  // MK_DECODE_STEP_TU
