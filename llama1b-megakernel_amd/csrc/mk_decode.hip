// mk_decode.hip — Llama-3.2-1B token-generation megakernel for MI355X (gfx950).
//
// One cooperative launch runs a whole decode step: for every decoder layer
//   QKV  : RMSNorm(h) -> [Wq;Wk;Wv] GEMV -> RoPE -> q, and K/V rows written
//          in place into the caches at row pos                 (attention.py:69-245, 450-492)
//   ATTN : GQA attention of the 32 q heads over K/V rows [0, pos], split over
//          the KV length, partial (max, sum, PV) merged by the last split to
//          finish each kv head                                 (attention.py:303-399)
//   O    : Wo GEMV + residual                                  (attention.py:409-448,
//                                                                transformer_llama.py:68-70)
//   GU   : RMSNorm(h1) -> gate/up GEMV -> silu(g)*u            (mlp.py:72-157)
//   DOWN : Wd GEMV + residual                                  (mlp.py:159-192,
//                                                                transformer_llama.py:82-84)
// then, optionally, the final RMSNorm, the tied lm_head GEMV and the greedy argmax.
//
// Design for CDNA4:
//   * one 256-thread workgroup (4 wave64s, one per SIMD) per CU, grid = #CUs,
//     launched cooperatively so all workgroups are co-resident;
//   * phases are separated by a grid barrier built from device-scope atomics:
//     each barrier has its own NCTR arrival counters on separate 128-byte
//     lines (one relaxed add per workgroup), wave 0 of each workgroup polls
//     them. There is no L2 writeback or invalidate at a barrier (an
//     agent-scope release/acquire costs ~10 us per phase on 8 XCDs): data a
//     workgroup hands to others is written with device-scope (sc1) stores,
//     each wave waits for its stores to complete (s_waitcnt vmcnt(0)) before
//     its workgroup arrives, every activation buffer is written once per launch
//     (one set per layer) so no XCD's L2 can hold a stale copy and readers
//     keep the L2 hits, and the one buffer rewritten within a launch (the
//     split-K partials) is read with device-scope loads;
//   * weights stream once from HBM through bounds-checked buffer loads
//     (16 B per lane, fully coalesced 1 KiB per wave per load); rows past a
//     wave's share are out-of-range offsets that return zero without a memory
//     access, so the software pipeline has no branches around its loads;
//   * before waiting at a barrier each wave has already issued the first
//     ring of the next phase's weight loads (they do not depend on the
//     activations), so the barrier latency overlaps HBM traffic;
//   * GEMVs are bf16 x bf16 -> fp32 with v_dot2_f32_bf16 and wave64
//     shuffle reductions (bs=1 is bandwidth-bound: no MFMA);
//   * the residual stream lives in two small global buffers that stay in
//     L2/MALL; every wave re-reads the full 4 KiB input vector and computes
//     RMSNorm for itself, so no extra barrier is needed for the norm.
#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "mk.h"

namespace {

constexpr int H = MK_HIDDEN;
constexpr int NQ = MK_N_Q_HEADS;
constexpr int NKV = MK_N_KV_HEADS;
constexpr int HD = MK_HEAD_DIM;
constexpr int GQA = NQ / NKV;
constexpr int INTER = MK_INTER;
constexpr int VOCAB = MK_VOCAB;
constexpr int QKV_ROWS = MK_QKV_ROWS;
constexpr int QKV_PAIRS = QKV_ROWS / 2;    // 1536 RoPE pairs
constexpr int Q_PAIRS = NQ * HD / 2;       // 1024
constexpr int K_PAIRS = NKV * HD / 2;      // 256
constexpr int NT = 256;                    // threads per workgroup
constexpr int NWAVE = NT / 64;
constexpr int ATT_MAX_SPLIT = 8;           // KV-length splits per kv head (attention work items)
constexpr int ATT_GROUP = 128;             // KV rows an attention item loads at once (4 rounds of 32)
constexpr int NCTR = 8;                    // arrival counters per grid barrier
constexpr int MAX_BARRIERS = 5 * MK_MAX_LAYERS + 4;
constexpr int CTR_STRIDE = 32;             // u32 words between counters (128 B)
constexpr int PART_FLOATS = GQA * (HD + 2);  // per split: m[4], l[4], o[4][64]
constexpr uint32_t OOB = 0x80000000u;      // buffer offset past every resource
constexpr float EPS = 1e-5f;
constexpr float SM_SCALE = 0.125f;         // 1/sqrt(64)
constexpr int MIN_GRID = 32;
constexpr int MAX_GRID = 1024;

constexpr size_t QKV_LAYER_BYTES = (size_t)QKV_ROWS * H * 2;
constexpr size_t O_LAYER_BYTES = (size_t)H * H * 2;
constexpr size_t GU_LAYER_BYTES = (size_t)2 * INTER * H * 2;
constexpr size_t D_LAYER_BYTES = (size_t)H * INTER * 2;
constexpr size_t EMBED_BYTES = (size_t)VOCAB * H * 2;

// Workspace layout (bytes, batch 1).
constexpr size_t OFF_BAR = 0;
constexpr size_t BAR_BYTES = (size_t)MAX_BARRIERS * NCTR * CTR_STRIDE * 4;
constexpr size_t OFF_MISC = BAR_BYTES;                 // exit counter, error bits, argmax key
constexpr size_t MISC_EXIT = 0, MISC_ERR = 1;                   // u32 indices
constexpr size_t MISC_KEY_BYTE = 128;                           // u64
// Activation buffers, one set per layer (each written once per launch):
//   h1 [2048] | q [2048] | att [2048] | act [8192] | h2 [2048]   (bf16)
constexpr size_t ACT_H1 = 0, ACT_Q = H * 2, ACT_ATT = 2 * H * 2, ACT_ACT = 3 * H * 2,
                 ACT_H2 = 3 * H * 2 + INTER * 2, ACT_LAYER_BYTES = 4 * H * 2 + INTER * 2;
constexpr size_t OFF_ACTS = OFF_MISC + 256;
// Split-K attention partials, one set per layer: [layer][kv head][split][m(4) l(4) o(4x64)] fp32.
constexpr size_t OFF_PART = OFF_ACTS + (size_t)MK_MAX_LAYERS * ACT_LAYER_BYTES;
constexpr size_t PART_LAYER_FLOATS = (size_t)NKV * ATT_MAX_SPLIT * PART_FLOATS;
constexpr size_t WS_BYTES = OFF_PART + (size_t)MK_MAX_LAYERS * PART_LAYER_FLOATS * 4;

inline size_t ws_bytes_for(int) { return WS_BYTES; }

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// fp32 -> bf16 bits, round to nearest even (NaN kept quiet).
__device__ __forceinline__ uint32_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float rbf(float f) { return __uint_as_float(f2bf(f) << 16); }
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) { return f2bf(lo) | (f2bf(hi) << 16); }

// 8-element bf16 dot product accumulated in fp32 (v_dot2_f32_bf16). The
// operands are bit-cast as whole 8-lane vectors and split with shufflevector:
// bit-casting individual u32 components to bf16x2 miscompiles (all four
// dot2 instructions end up reading the same register pair).
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
__device__ __forceinline__ float dot8(u32x4 a, u32x4 b, float acc) {
  const bf16x8_t A = __builtin_bit_cast(bf16x8_t, a), B = __builtin_bit_cast(bf16x8_t, b);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(A, A, 0, 1), __builtin_shufflevector(B, B, 0, 1), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(A, A, 2, 3), __builtin_shufflevector(B, B, 2, 3), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(A, A, 4, 5), __builtin_shufflevector(B, B, 4, 5), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(A, A, 6, 7), __builtin_shufflevector(B, B, 6, 7), acc, false);
  return acc;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

constexpr int AUX_NT = 2, AUX_SC1 = 16;   // buffer-load cache policy bits (gfx950)

__device__ __forceinline__ rsrc_t make_rsrc(const void* p, size_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
// Streaming 16-byte load (non-temporal); offsets >= the resource size read zero.
__device__ __forceinline__ u32x4 ld_stream(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, AUX_NT);
}

// Device-scope (sc1) accesses for data exchanged between workgroups within a
// launch: the store writes through to the device coherence point, the load
// never returns a line cached before that point was updated.
__device__ __forceinline__ void st_dev(uint16_t* p, uint32_t bf_bits) {
  __hip_atomic_store(p, (uint16_t)bf_bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u32x4 ld_dev16(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, AUX_SC1);
}
// Completion of this wave's outstanding memory operations (stores included).
__device__ __forceinline__ void wait_mem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

// Contiguous share [lo, hi) of `total` items for part `i` of `n`.
__device__ __forceinline__ void share(int total, int n, int i, int& lo, int& hi) {
  lo = (int)(((long long)total * i) / n);
  hi = (int)(((long long)total * (i + 1)) / n);
}

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
  int first_layer;
  int n_layers;
  int s_max;
  int rope_rows;
  int do_lm;
  uint32_t flags;
  unsigned long long timeout_ticks;
  unsigned long long* trace;
};

// ---------------------------------------------------------------------------
// Grid barrier: per-barrier counters, split arrive / wait.
// ---------------------------------------------------------------------------
struct Grid {
  uint32_t* bar;
  uint32_t* err;
  int G;
  int wg;
  int k;                       // number of arrivals issued so far
  unsigned long long timeout;
  unsigned long long* trace;   // this workgroup's MK_TRACE_SLOTS slots, or null
};

__device__ __forceinline__ void trace_mark(const Grid& g, int slot) {
  if (g.trace && threadIdx.x == 0 && slot < MK_TRACE_SLOTS) g.trace[slot] = wall_clock64();
}

// Arrive: every wave's stores are complete, then one relaxed add per workgroup.
__device__ __forceinline__ void grid_arrive(Grid& g) {
  wait_mem();
  __syncthreads();
  if (threadIdx.x == 0)
    __hip_atomic_fetch_add(g.bar + ((size_t)g.k * NCTR + (g.wg % NCTR)) * CTR_STRIDE, 1u,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  ++g.k;
  trace_mark(g, 2 * g.k - 1);
}

// Wait until every workgroup has arrived at barrier `k` (0-based). Wave 0
// polls; the other waves wait at the workgroup barrier without draining their
// in-flight weight loads.
__device__ __forceinline__ void grid_wait_k(const Grid& g, int k) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const int c = lane < NCTR ? lane : 0;
    const uint32_t need = lane < NCTR ? (uint32_t)(g.G / NCTR + (lane < g.G % NCTR ? 1 : 0)) : 0u;
    uint32_t* a = g.bar + ((size_t)k * NCTR + c) * CTR_STRIDE;
    const unsigned long long t0 = wall_clock64();
    while (true) {
      const uint32_t v = __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (__all(v >= need)) break;
      const uint32_t e = __hip_atomic_load(g.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (e & MK_DEVERR_BARRIER) break;
      if (wall_clock64() - t0 > g.timeout) {
        if (lane == 0)
          __hip_atomic_fetch_or(g.err, MK_DEVERR_BARRIER, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  __syncthreads();
}

// Wait on the latest barrier this workgroup arrived at.
__device__ __forceinline__ void grid_wait(Grid& g) {
  grid_wait_k(g, g.k - 1);
  trace_mark(g, 2 * g.k);
}

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
  __device__ __forceinline__ void issue(int slot_row, u32x4 (&dst)[KCH]) const {
    const uint32_t o = row_off(slot_row) + (uint32_t)lane_id() * 16u;
#pragma unroll
    for (int i = 0; i < KCH; ++i) dst[i] = ld_stream(rs, o + (uint32_t)i * 1024u);
  }
  __device__ __forceinline__ void start(rsrc_t r, uint32_t o0, uint32_t st, int count) {
    rs = r;
    off0 = o0;
    stride = st;
    n = count;
#pragma unroll
    for (int j = 0; j < RING; ++j) issue(j, buf[j]);
  }
  // dotf(buf) -> partial (per lane); emit(r, partial) for each valid row r.
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
  }
};

// The wave's rows of a workgroup share [lo, hi): lo + wave + 4*j.
__device__ __forceinline__ int wave_count(int lo, int hi) {
  const int n = hi - lo - wave_id();
  return n > 0 ? (n + NWAVE - 1) / NWAVE : 0;
}

// Lane slice of a 2048-vector: elements i*512 + lane*8 .. +7.
__device__ __forceinline__ void load_x2048(const uint16_t* x, u32x4 (&xs)[4]) {
  const int lane = lane_id();
#pragma unroll
  for (int i = 0; i < 4; ++i) xs[i] = *reinterpret_cast<const u32x4*>(x + i * 512 + lane * 8);
}

// In-register RMSNorm of the wave's full 2048-vector copy:
//   xn = bf16(x * rsqrt(mean(x^2) + eps))            (gamma folded into the weights)
//   xn = bf16(g * bf16(x * rsqrt(mean(x^2) + eps)))  (final norm, HF LlamaRMSNorm)
__device__ __forceinline__ void rmsnorm2048(u32x4 (&xs)[4], const uint16_t* gamma) {
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w[4] = {xs[i].x, xs[i].y, xs[i].z, xs[i].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = bf_lo(w[j]), b = bf_hi(w[j]);
      ss = fmaf(a, a, ss);
      ss = fmaf(b, b, ss);
    }
  }
  ss = wave_sum(ss);
  const float inv = rsqrtf(ss * (1.0f / H) + EPS);
  const int lane = lane_id();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t w[4] = {xs[i].x, xs[i].y, xs[i].z, xs[i].w};
    u32x4 gv = {0u, 0u, 0u, 0u};
    if (gamma) gv = *reinterpret_cast<const u32x4*>(gamma + i * 512 + lane * 8);
    const uint32_t g[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float a = rbf(bf_lo(w[j]) * inv), b = rbf(bf_hi(w[j]) * inv);
      if (gamma) {
        a = bf_lo(g[j]) * a;
        b = bf_hi(g[j]) * b;
      }
      w[j] = pack_bf2(a, b);
    }
    xs[i] = u32x4{w[0], w[1], w[2], w[3]};
  }
}

// ---------------------------------------------------------------------------
// The megakernel
// ---------------------------------------------------------------------------
struct Ctx {
  const KParams* p;
  Grid g;
  int pos;
  int n_rows;            // KV rows attended: pos + 1
  const uint16_t* x_in;  // input of the first layer (embedding row or hidden_in)
  uint8_t* acts;         // per-layer activation buffers
  float* part;
  uint32_t* misc;

  __device__ __forceinline__ uint16_t* buf(int li, size_t which) const {
    return reinterpret_cast<uint16_t*>(acts + (size_t)li * ACT_LAYER_BYTES + which);
  }
  // layer input: the previous layer's h2, or the step input for the first layer
  __device__ __forceinline__ const uint16_t* h_in(int li) const { return li == 0 ? x_in : buf(li - 1, ACT_H2); }
};

__device__ __forceinline__ u32x4 rope_pair(float a, float b, const uint16_t* rrow, int d) {
  // out[d]    = bf16(bf16(a*cos[d])    + bf16(-b*sin[d]))
  // out[d+32] = bf16(bf16(b*cos[d+32]) + bf16( a*sin[d+32]))      (attention.py:160-174)
  const float c0 = bf2f(rrow[d]), c1 = bf2f(rrow[d + 32]);
  const float s0 = bf2f(rrow[64 + d]), s1 = bf2f(rrow[64 + d + 32]);
  const float ra = rbf(rbf(a * c0) + rbf(-b * s0));
  const float rb = rbf(rbf(b * c1) + rbf(a * s1));
  return u32x4{f2bf(ra), f2bf(rb), 0u, 0u};
}

// QKV phase of run-layer li (stack layer l): RMSNorm, GEMV, RoPE, q out, K/V rows in place.
__device__ __forceinline__ void phase_qkv(Ctx& c, int li, float* s_val) {
  const KParams& p = *c.p;
  const int l = p.first_layer + li;
  const int G = c.g.G, w = c.g.wg, wave = wave_id();
  int P0, P1;
  share(QKV_PAIRS, G, w, P0, P1);
  const int nrows = 2 * (P1 - P0);
  RowStream<4, 4> rs;
  rs.start(make_rsrc(p.w_qkv + (size_t)l * QKV_ROWS * H, QKV_LAYER_BYTES),
           (uint32_t)(2 * P0 + wave) * (H * 2), NWAVE * H * 2, wave_count(0, nrows));
  if (li > 0) grid_wait(c.g);
  u32x4 xs[4];
  load_x2048(c.h_in(li), xs);
  rmsnorm2048(xs, nullptr);
  rs.run([&](const u32x4(&wv)[4]) {
           float a = dot8(wv[0], xs[0], 0.f);
           float b = dot8(wv[1], xs[1], 0.f);
           a = dot8(wv[2], xs[2], a);
           b = dot8(wv[3], xs[3], b);
           return a + b;
         },
         [&](int r, float part) {
           const float v = wave_sum(part);
           if (lane_id() == 0) s_val[wave + NWAVE * r] = v;
         });
  __syncthreads();
  const uint16_t* rrow = p.rope + (size_t)c.pos * (2 * HD);
  uint16_t* qv = c.buf(li, ACT_Q);
  for (int lp = threadIdx.x; lp < P1 - P0; lp += NT) {
    const int pr = P0 + lp;
    const float a = rbf(s_val[2 * lp]), b = rbf(s_val[2 * lp + 1]);
    uint16_t* dst;
    u32x4 o;
    if (pr < Q_PAIRS) {
      dst = qv + (pr >> 5) * HD;
      o = rope_pair(a, b, rrow, pr & 31);
    } else if (pr < Q_PAIRS + K_PAIRS) {
      dst = p.kc[li] + ((size_t)((pr - Q_PAIRS) >> 5) * p.s_max + c.pos) * HD;
      o = rope_pair(a, b, rrow, pr & 31);
    } else {
      dst = p.vc[li] + ((size_t)((pr - Q_PAIRS - K_PAIRS) >> 5) * p.s_max + c.pos) * HD;
      o = u32x4{f2bf(a), f2bf(b), 0u, 0u};
    }
    st_dev(dst + (pr & 31), o.x);
    st_dev(dst + (pr & 31) + 32, o.y);
  }
  grid_arrive(c.g);
}

// One attention work item: kv head h, KV rows [j0, j1) of [0, n_rows), for the
// 4 q heads of the group (GQA). Thread t serves row (t >> 3) of each 32-row
// round and the 8 dims (t & 7)*8.. of it; rows stream in groups of
// ATT_GROUP with an online softmax. Writes the item's partial
// (m[4], l[4], o[4][64]) unnormalised, relative to m.
struct AttnShared {
  float mx[NWAVE][GQA];
  float sm[NWAVE][GQA];
  float pv[NWAVE][8][GQA * 8];
};

__device__ __forceinline__ void attn_item(Ctx& c, int li, int h, int j0, int j1, float* part, AttnShared& sh) {
  const KParams& p = *c.p;
  const int t = threadIdx.x, rl = t >> 3, ch = t & 7, wave = wave_id(), lane = lane_id();
  // this head's K and V rows, device-scope loads (row pos was written in this launch)
  const size_t head_bytes = (size_t)p.s_max * HD * 2;
  const rsrc_t rk = make_rsrc(p.kc[li] + (size_t)h * p.s_max * HD, head_bytes);
  const rsrc_t rv = make_rsrc(p.vc[li] + (size_t)h * p.s_max * HD, head_bytes);
  const uint16_t* qv = c.buf(li, ACT_Q);
  u32x4 q[GQA];
#pragma unroll
  for (int g = 0; g < GQA; ++g) q[g] = *reinterpret_cast<const u32x4*>(qv + (h * GQA + g) * HD + ch * 8);
  float m_run[GQA], l_run[GQA], acc[GQA][8];
#pragma unroll
  for (int g = 0; g < GQA; ++g) {
    m_run[g] = -INFINITY;
    l_run[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  }
  constexpr int R = ATT_GROUP / 32;
  for (int base = j0; base < j1; base += ATT_GROUP) {
    u32x4 kk[R], vv[R];
    bool valid[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int j = base + 32 * r + rl;
      valid[r] = j < j1;
      const uint32_t off = valid[r] ? (uint32_t)(j * HD + ch * 8) * 2u : OOB;
      kk[r] = ld_dev16(rk, off);
      vv[r] = ld_dev16(rv, off);
    }
    float sc[R][GQA];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int g = 0; g < GQA; ++g) {
        float x = dot8(kk[r], q[g], 0.f);
        x += __shfl_xor(x, 1, 64);
        x += __shfl_xor(x, 2, 64);
        x += __shfl_xor(x, 4, 64);
        sc[r][g] = valid[r] ? x * SM_SCALE : -INFINITY;
      }
#pragma unroll
    for (int g = 0; g < GQA; ++g) {
      float mn = m_run[g];
#pragma unroll
      for (int r = 0; r < R; ++r) mn = fmaxf(mn, sc[r][g]);
      const float keep = mn == -INFINITY ? 1.f : __expf(m_run[g] - mn);
      l_run[g] *= keep;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] *= keep;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float pr = valid[r] ? __expf(sc[r][g] - mn) : 0.f;
        l_run[g] += pr;
        const uint32_t w4[4] = {vv[r].x, vv[r].y, vv[r].z, vv[r].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[g][2 * e] = fmaf(pr, bf_lo(w4[e]), acc[g][2 * e]);
          acc[g][2 * e + 1] = fmaf(pr, bf_hi(w4[e]), acc[g][2 * e + 1]);
        }
      }
      m_run[g] = mn;
    }
  }
  // merge the 32 row-lanes of the item: max, rescale, sum (lanes of one row agree)
#pragma unroll
  for (int g = 0; g < GQA; ++g) {
    float m = m_run[g];
    m = fmaxf(m, __shfl_xor(m, 8, 64));
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    if (lane == 0) sh.mx[wave][g] = m;
  }
  __syncthreads();
#pragma unroll
  for (int g = 0; g < GQA; ++g) {
    const float M = fmaxf(fmaxf(sh.mx[0][g], sh.mx[1][g]), fmaxf(sh.mx[2][g], sh.mx[3][g]));
    const float f = m_run[g] == -INFINITY ? 0.f : __expf(m_run[g] - M);
    float l = l_run[g] * f;
    l += __shfl_xor(l, 8, 64);
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    if (lane == 0) sh.sm[wave][g] = l;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = acc[g][e] * f;
      v += __shfl_xor(v, 8, 64);
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      acc[g][e] = v;
    }
  }
  if (lane < 8) {
#pragma unroll
    for (int g = 0; g < GQA; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) sh.pv[wave][ch][g * 8 + e] = acc[g][e];
  }
  __syncthreads();
  {
    const int g = t >> 6, d = t & 63;
    float o = 0.f;
#pragma unroll
    for (int wv = 0; wv < NWAVE; ++wv) o += sh.pv[wv][d >> 3][g * 8 + (d & 7)];
    st_dev(part + 2 * GQA + g * HD + d, o);
    if (t < GQA) {
      st_dev(part + t, fmaxf(fmaxf(sh.mx[0][t], sh.mx[1][t]), fmaxf(sh.mx[2][t], sh.mx[3][t])));
      st_dev(part + GQA + t, sh.sm[0][t] + sh.sm[1][t] + sh.sm[2][t] + sh.sm[3][t]);
    }
  }
  __syncthreads();   // LDS reuse by a following item
}

// Split of [0, n_rows) into nsplit items of `rows` rows (a multiple of 32).
__device__ __forceinline__ void attn_split(int n_rows, int& nsplit, int& rows) {
  int ns = (n_rows + 31) / 32;
  ns = ns < ATT_MAX_SPLIT ? ns : ATT_MAX_SPLIT;
  rows = ((n_rows + ns - 1) / ns + 31) / 32 * 32;
  nsplit = (n_rows + rows - 1) / rows;
}

// Merge the split-K partials of all 32 q heads into bf16 att in LDS:
//   att = sum_s e^(m_s-M) o_s / sum_s e^(m_s-M) l_s   (then cast to bf16)
// Thread t produces q head t>>3, dims (t&7)*8 .. +7.
__device__ __forceinline__ void attn_merge(const float* part_layer, int nsplit, uint16_t* att_lds) {
  const int t = threadIdx.x, qh = t >> 3, d0 = (t & 7) * 8, h = qh >> 2, g = qh & 3;
  // all loads issued at once; splits >= nsplit read zero through out-of-range offsets
  const rsrc_t r = make_rsrc(part_layer + (size_t)h * ATT_MAX_SPLIT * PART_FLOATS,
                             (size_t)nsplit * PART_FLOATS * 4);
  u32x4 ml[ATT_MAX_SPLIT][2], oa[ATT_MAX_SPLIT], ob[ATT_MAX_SPLIT];
#pragma unroll
  for (int s = 0; s < ATT_MAX_SPLIT; ++s) {
    const uint32_t base = (uint32_t)(s * PART_FLOATS) * 4u;
    ml[s][0] = __builtin_amdgcn_raw_buffer_load_b128(r, (int)base, 0, 0);          // m[0..3]
    ml[s][1] = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(base + 16u), 0, 0);  // l[0..3]
    const uint32_t o = base + (uint32_t)(2 * GQA + g * HD + d0) * 4u;
    oa[s] = __builtin_amdgcn_raw_buffer_load_b128(r, (int)o, 0, 0);
    ob[s] = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(o + 16u), 0, 0);
  }
  auto pick = [g](u32x4 v) { return __uint_as_float(g == 0 ? v.x : g == 1 ? v.y : g == 2 ? v.z : v.w); };
  float M = -INFINITY;
#pragma unroll
  for (int s = 0; s < ATT_MAX_SPLIT; ++s)
    if (s < nsplit) M = fmaxf(M, pick(ml[s][0]));
  float O[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float L = 0.f;
#pragma unroll
  for (int s = 0; s < ATT_MAX_SPLIT; ++s) {
    const float w = s < nsplit ? __expf(pick(ml[s][0]) - M) : 0.f;
    L = fmaf(w, pick(ml[s][1]), L);
    O[0] = fmaf(w, __uint_as_float(oa[s].x), O[0]);
    O[1] = fmaf(w, __uint_as_float(oa[s].y), O[1]);
    O[2] = fmaf(w, __uint_as_float(oa[s].z), O[2]);
    O[3] = fmaf(w, __uint_as_float(oa[s].w), O[3]);
    O[4] = fmaf(w, __uint_as_float(ob[s].x), O[4]);
    O[5] = fmaf(w, __uint_as_float(ob[s].y), O[5]);
    O[6] = fmaf(w, __uint_as_float(ob[s].z), O[6]);
    O[7] = fmaf(w, __uint_as_float(ob[s].w), O[7]);
  }
  const float inv = 1.0f / L;
  u32x4 out;
  out.x = pack_bf2(O[0] * inv, O[1] * inv);
  out.y = pack_bf2(O[2] * inv, O[3] * inv);
  out.z = pack_bf2(O[4] * inv, O[5] * inv);
  out.w = pack_bf2(O[6] * inv, O[7] * inv);
  *reinterpret_cast<u32x4*>(att_lds + qh * HD + d0) = out;
}

__global__ void __launch_bounds__(NT, 1) mk_decode_kernel(KParams p) {
  __shared__ float s_val[128];
  __shared__ AttnShared s_att;
  __shared__ __attribute__((aligned(16))) uint16_t s_attv[H];
  __shared__ float s_best[NWAVE];
  __shared__ int s_bidx[NWAVE];
  __shared__ int s_last;

  Ctx c;
  c.p = &p;
  c.g.bar = reinterpret_cast<uint32_t*>(p.ws + OFF_BAR);
  c.misc = reinterpret_cast<uint32_t*>(p.ws + OFF_MISC);
  c.g.err = c.misc + MISC_ERR;
  c.g.G = gridDim.x;
  c.g.wg = blockIdx.x;
  c.g.k = 0;
  c.g.timeout = p.timeout_ticks;
  c.g.trace = p.trace ? p.trace + (size_t)blockIdx.x * MK_TRACE_SLOTS : nullptr;
  trace_mark(c.g, 0);
  c.acts = p.ws + OFF_ACTS;
  c.part = reinterpret_cast<float*>(p.ws + OFF_PART);
  c.pos = p.pos[0];
  const bool pos_ok = c.pos >= 0 && c.pos < p.s_max && c.pos < p.rope_rows;
  if (!pos_ok && blockIdx.x == 0 && threadIdx.x == 0)
    __hip_atomic_fetch_or(c.g.err, MK_DEVERR_POS, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  c.n_rows = c.pos + 1;
  if (p.hidden_in) {
    c.x_in = p.hidden_in;
  } else {
    int tok = p.tokens[0];
    tok = tok < 0 ? 0 : (tok >= VOCAB ? VOCAB - 1 : tok);
    c.x_in = p.embed + (size_t)tok * H;
  }
  const int G = c.g.G, w = c.g.wg, wave = wave_id(), lane = lane_id();

  if (pos_ok) {
    int R0, R1;
    share(H, G, w, R0, R1);
    for (int li = 0; li < p.n_layers; ++li) {
      const int l = p.first_layer + li;
      const bool last = li == p.n_layers - 1;
      phase_qkv(c, li, s_val);

      // ---- attention; the O-projection weights are prefetched meanwhile ----
      RowStream<2, 4> os;
      int nsplit, rows;
      attn_split(c.n_rows, nsplit, rows);
      const int nitems = NKV * nsplit;
      float* part_l = c.part + (size_t)li * PART_LAYER_FLOATS;
      if (w < nitems) {
        os.start(make_rsrc(p.w_o + (size_t)l * H * H, O_LAYER_BYTES), (uint32_t)(R0 + wave) * (H * 2),
                 NWAVE * H * 2, wave_count(R0, R1));
        grid_wait(c.g);
        for (int it = w; it < nitems; it += G) {
          const int h = it / nsplit, sp = it % nsplit;
          const int j0 = sp * rows, j1 = min(j0 + rows, c.n_rows);
          attn_item(c, li, h, j0, j1, part_l + ((size_t)h * ATT_MAX_SPLIT + sp) * PART_FLOATS, s_att);
        }
        grid_arrive(c.g);
      } else {
        // no attention work: arrive at once without waiting on the QKV
        // barrier (each barrier has its own counters, so arriving early is safe)
        grid_arrive(c.g);
        os.start(make_rsrc(p.w_o + (size_t)l * H * H, O_LAYER_BYTES), (uint32_t)(R0 + wave) * (H * 2),
                 NWAVE * H * 2, wave_count(R0, R1));
      }

      // ---- O projection + residual -> h1 ----
      grid_wait(c.g);
      attn_merge(part_l, nsplit, s_attv);
      __syncthreads();
      {
        u32x4 xs[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) xs[i] = *reinterpret_cast<const u32x4*>(s_attv + i * 512 + lane * 8);
        const uint16_t* hprev = c.h_in(li);
        uint16_t* h1 = c.buf(li, ACT_H1);
        os.run([&](const u32x4(&wv)[4]) {
                 float a = dot8(wv[0], xs[0], 0.f);
                 float b = dot8(wv[1], xs[1], 0.f);
                 a = dot8(wv[2], xs[2], a);
                 b = dot8(wv[3], xs[3], b);
                 return a + b;
               },
               [&](int r, float part) {
                 const float v = wave_sum(part);
                 if (lane == 0) {
                   const int row = R0 + wave + NWAVE * r;
                   st_dev(h1 + row, f2bf(bf2f(hprev[row]) + rbf(v)));
                 }
               });
      }
      grid_arrive(c.g);

      // ---- gate/up + SwiGLU -> act ----
      {
        int U0, U1;
        share(INTER, G, w, U0, U1);
        RowStream<4, 8> gs;
        gs.start(make_rsrc(p.w_gu + (size_t)l * 2 * INTER * H, GU_LAYER_BYTES),
                 (uint32_t)(U0 + wave) * (2 * H * 2), NWAVE * 2 * H * 2, wave_count(U0, U1));
        grid_wait(c.g);
        u32x4 xs[4];
        load_x2048(c.buf(li, ACT_H1), xs);
        rmsnorm2048(xs, nullptr);
        uint16_t* act = c.buf(li, ACT_ACT);
        struct GU2 { float g, u; };
        gs.run([&](const u32x4(&wv)[8]) {
                 float g0 = dot8(wv[0], xs[0], 0.f), g1 = dot8(wv[1], xs[1], 0.f);
                 float u0 = dot8(wv[4], xs[0], 0.f), u1 = dot8(wv[5], xs[1], 0.f);
                 g0 = dot8(wv[2], xs[2], g0);
                 g1 = dot8(wv[3], xs[3], g1);
                 u0 = dot8(wv[6], xs[2], u0);
                 u1 = dot8(wv[7], xs[3], u1);
                 return GU2{g0 + g1, u0 + u1};
               },
               [&](int r, GU2 part) {
                 const float gv = wave_sum(part.g);
                 const float uv = wave_sum(part.u);
                 if (lane == 0) {
                   const float silu = gv / (1.0f + __expf(-gv));
                   st_dev(act + U0 + wave + NWAVE * r, f2bf(silu * uv));
                 }
               });
      }
      grid_arrive(c.g);

      // ---- down projection + residual -> h2 ----
      {
        RowStream<2, 16> ds;
        ds.start(make_rsrc(p.w_d + (size_t)l * H * INTER, D_LAYER_BYTES), (uint32_t)(R0 + wave) * (INTER * 2),
                 NWAVE * INTER * 2, wave_count(R0, R1));
        grid_wait(c.g);
        const uint16_t* act = c.buf(li, ACT_ACT);
        const uint16_t* h1 = c.buf(li, ACT_H1);
        uint16_t* h2 = c.buf(li, ACT_H2);
        u32x4 xs[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) xs[i] = *reinterpret_cast<const u32x4*>(act + i * 512 + lane * 8);
        ds.run([&](const u32x4(&wv)[16]) {
                 float a = 0.f, b = 0.f;
#pragma unroll
                 for (int i = 0; i < 16; i += 2) {
                   a = dot8(wv[i], xs[i], a);
                   b = dot8(wv[i + 1], xs[i + 1], b);
                 }
                 return a + b;
               },
               [&](int r, float part) {
                 const float v = wave_sum(part);
                 if (lane == 0) {
                   const int row = R0 + wave + NWAVE * r;
                   const uint32_t hv = f2bf(bf2f(h1[row]) + rbf(v));
                   st_dev(h2 + row, hv);
                   if (last && p.hidden_out) p.hidden_out[row] = (uint16_t)hv;
                 }
               });
      }
      grid_arrive(c.g);
    }

    // ---- final norm + tied lm_head + argmax ----
    if (p.do_lm) {
      int V0, V1;
      share(VOCAB, G, w, V0, V1);
      RowStream<8, 4> ls;
      ls.start(make_rsrc(p.embed, EMBED_BYTES), (uint32_t)(V0 + wave) * (H * 2), NWAVE * H * 2,
               wave_count(V0, V1));
      grid_wait(c.g);
      u32x4 xs[4];
      load_x2048(c.buf(p.n_layers - 1, ACT_H2), xs);
      rmsnorm2048(xs, p.g_final);
      float best = -INFINITY;
      int bidx = 0x7fffffff;
      ls.run([&](const u32x4(&wv)[4]) {
               float a = dot8(wv[0], xs[0], 0.f);
               float b = dot8(wv[1], xs[1], 0.f);
               a = dot8(wv[2], xs[2], a);
               b = dot8(wv[3], xs[3], b);
               return a + b;
             },
             [&](int r, float part) {
               const float v = wave_sum(part);
               const int row = V0 + wave + NWAVE * r;
               if (lane == 0 && p.logits) p.logits[row] = v;
               if (v > best) {   // rows ascend: keeps the lowest index among equal maxima
                 best = v;
                 bidx = row;
               }
             });
      if (lane == 0) {
        s_best[wave] = best;
        s_bidx[wave] = bidx;
      }
      __syncthreads();
      if (threadIdx.x == 0) {
        float b = s_best[0];
        int bi = s_bidx[0];
        for (int k = 1; k < NWAVE; ++k)
          if (s_best[k] > b || (s_best[k] == b && s_bidx[k] < bi)) {
            b = s_best[k];
            bi = s_bidx[k];
          }
        if (bi != 0x7fffffff) {
          uint32_t u = __float_as_uint(b);
          u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);   // order-preserving float key
          const unsigned long long key =
              ((unsigned long long)u << 32) | (unsigned long long)(0xffffffffu - (uint32_t)bi);
          __hip_atomic_fetch_max(reinterpret_cast<unsigned long long*>(p.ws + OFF_MISC + MISC_KEY_BYTE), key,
                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
  }

  // ---- exit: the last workgroup out finalises and resets the control block ----
  trace_mark(c.g, MK_TRACE_SLOTS - 1);
  wait_mem();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev =
        __hip_atomic_fetch_add(c.misc + MISC_EXIT, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == (uint32_t)(G - 1);
  }
  __syncthreads();
  if (!s_last) return;
  for (int i = threadIdx.x; i < c.g.k * NCTR; i += NT) c.g.bar[(size_t)i * CTR_STRIDE] = 0u;
  if (threadIdx.x == 0) {
    c.misc[MISC_EXIT] = 0u;
    if (pos_ok) {
      if (p.do_lm) {
        unsigned long long* kp = reinterpret_cast<unsigned long long*>(p.ws + OFF_MISC + MISC_KEY_BYTE);
        const unsigned long long key = __hip_atomic_load(kp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *kp = 0ull;
        if (p.next_token) p.next_token[0] = (int32_t)(0xffffffffu - (uint32_t)(key & 0xffffffffull));
      }
      if (p.flags & MK_FLAG_ADVANCE) p.pos[0] = c.pos + 1;
    }
  }
}

__global__ void mk_zero_kernel(u32x4* p, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = u32x4{0u, 0u, 0u, 0u};
}

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
  int grid;
  unsigned long long ticks_per_s;
  int status;
};
DeviceInfo g_dev[64];
std::mutex g_dev_mu;

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
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void*>(mk_decode_kernel), NT, 0) !=
        hipSuccess)
      return fail(MK_ERR_HIP, "occupancy query failed");
    d.grid = cus;
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

}  // namespace

extern "C" {

int mk_abi_version(void) { return MK_ABI_VERSION; }

const char* mk_last_error(void) { return g_msg; }

int mk_grid_size(int device) {
  DeviceInfo d;
  const int rc = device_info(device, &d);
  return rc == MK_OK ? d.grid : rc;
}

long long mk_wall_clock_hz(int device) {
  DeviceInfo d;
  const int rc = device_info(device, &d);
  return rc == MK_OK ? (long long)d.ticks_per_s : rc;
}

size_t mk_workspace_bytes(int32_t batch, int32_t s_max) {
  if (batch != 1 || s_max < 1 || s_max > (1 << 20)) return 0;
  return ws_bytes_for(s_max);
}

int mk_workspace_init(void* workspace, size_t workspace_bytes, void* stream) {
  if (!workspace) return fail(MK_ERR_NULL, "workspace is NULL");
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) || (workspace_bytes & 15u))
    return fail(MK_ERR_WORKSPACE, "workspace must be 256-byte aligned with a size multiple of 16");
  const size_t n = workspace_bytes / 16;
  const int blocks = (int)((n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024);
  hipLaunchKernelGGL(mk_zero_kernel, dim3(blocks > 0 ? blocks : 1), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<u32x4*>(workspace), n);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MK_ERR_HIP, "zero kernel launch: %s", hipGetErrorString(e));
  return MK_OK;
}

int mk_read_device_error(void* workspace, void* stream, uint32_t* bits_out) {
  if (!workspace || !bits_out) return fail(MK_ERR_NULL, "workspace or bits_out is NULL");
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e = hipStreamSynchronize(st);
  if (e != hipSuccess) return fail(MK_ERR_HIP, "hipStreamSynchronize: %s", hipGetErrorString(e));
  uint32_t* dev_err = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(workspace) + OFF_MISC) + MISC_ERR;
  uint32_t bits = 0, zero = 0;
  e = hipMemcpy(&bits, dev_err, 4, hipMemcpyDeviceToHost);
  if (e == hipSuccess) e = hipMemcpy(dev_err, &zero, 4, hipMemcpyHostToDevice);
  if (e != hipSuccess) return fail(MK_ERR_HIP, "reading device error: %s", hipGetErrorString(e));
  *bits_out = bits;
  return MK_OK;
}

int mk_decode_step(const mk_weights* w, const mk_step_args* a) {
  if (!w || !a) return fail(MK_ERR_NULL, "weights or args is NULL");
  if (a->n_layers < 1 || a->first_layer < 0 || a->first_layer + a->n_layers > w->n_layers ||
      w->n_layers > MK_MAX_LAYERS)
    return fail(MK_ERR_SHAPE, "layers [%d, %d) not within the %d packed layers (max %d)", a->first_layer,
                a->first_layer + a->n_layers, w->n_layers, MK_MAX_LAYERS);
  if (a->batch < 1) return fail(MK_ERR_SHAPE, "batch %d < 1", a->batch);
  if (a->batch != 1) return fail(MK_ERR_UNSUPPORTED, "batch %d: this build runs batch 1", a->batch);
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
  if (!a->workspace) return fail(MK_ERR_NULL, "workspace is NULL");
  if (reinterpret_cast<uintptr_t>(a->workspace) & 255u) return fail(MK_ERR_WORKSPACE, "workspace not 256-byte aligned");
  const size_t need = mk_workspace_bytes(a->batch, a->s_max);
  if (a->workspace_bytes < need)
    return fail(MK_ERR_WORKSPACE, "workspace %zu bytes < %zu needed", a->workspace_bytes, need);

  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(MK_ERR_HIP, "hipGetDevice failed");
  DeviceInfo di;
  const int rc = device_info(dev, &di);
  if (rc != MK_OK) return rc;

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
  kp.ws = static_cast<uint8_t*>(a->workspace);
  kp.first_layer = a->first_layer;
  kp.n_layers = a->n_layers;
  kp.s_max = a->s_max;
  kp.rope_rows = w->rope_rows;
  kp.do_lm = do_lm ? 1 : 0;
  kp.flags = a->flags;
  kp.timeout_ticks = di.ticks_per_s * 2ull;   // 2 s per barrier wait
  kp.trace = static_cast<unsigned long long*>(a->trace);

  void* args[] = {&kp};
  const hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(mk_decode_kernel), dim3(di.grid),
                                                  dim3(NT), args, 0, static_cast<hipStream_t>(a->stream));
  if (e != hipSuccess) return fail(MK_ERR_HIP, "cooperative launch failed: %s", hipGetErrorString(e));
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
