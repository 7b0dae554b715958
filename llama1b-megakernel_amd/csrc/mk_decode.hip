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

// Workspace (bytes, batch 1): a control block. The two sets of exchange buffers
// live in a separate uncached area (SET_BYTES each) tied to the workspace.
constexpr size_t CTRL_BYTES = 256;
constexpr int C_EXIT = 0, C_ERR = 1, C_EPOCH = 2;   // u32 words of the control block
constexpr size_t C_KEY_BYTE = 128;                  // u64 argmax key
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

inline size_t ws_bytes_for(int) { return WS_BYTES; }

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// fp32 -> bf16 bits, round to nearest even. Every NaN becomes the canonical
// quiet NaN 0x7fc0, so the exchange sentinel 0xffff is never produced.
__device__ __forceinline__ uint32_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float rbf(float f) { return __uint_as_float(f2bf(f) << 16); }
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) { return f2bf(lo) | (f2bf(hi) << 16); }
// fp32 for an exchange buffer: NaN canonicalised (never the 0xffffffff sentinel).
__device__ __forceinline__ float canon(float f) { return f != f ? __uint_as_float(0x7fc00000u) : f; }

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

// Cross-lane moves. DPP (data-parallel primitives) read a neighbour lane's
// register within the same instruction; readlane copies one lane to a scalar.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float lane_val(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
constexpr int DPP_XOR1 = 0xb1;      // quad_perm [1,0,3,2]
constexpr int DPP_XOR2 = 0x4e;      // quad_perm [2,3,0,1]
constexpr int DPP_ROR4 = 0x124;     // row_ror:4 (rotate within 16 lanes)
constexpr int DPP_ROR8 = 0x128;     // row_ror:8

// Sum over the 64 lanes, returned in every lane.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<DPP_XOR1>(v);
  v += dpp<DPP_XOR2>(v);
  v += dpp<DPP_ROR4>(v);
  v += dpp<DPP_ROR8>(v);     // every lane now holds the sum of its 16-lane row
  return (lane_val(v, 0) + lane_val(v, 16)) + (lane_val(v, 32) + lane_val(v, 48));
}

constexpr int AUX_NT = 2, AUX_SC1 = 16;   // buffer-load cache policy bits (gfx950)

__device__ __forceinline__ rsrc_t make_rsrc(const void* p, size_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
// Streaming 16-byte load (non-temporal); offsets >= the resource size read zero.
__device__ __forceinline__ u32x4 ld_stream(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, AUX_NT);
}
__device__ __forceinline__ u32x4 ld16(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
}

// Device-scope (sc1) accesses for data exchanged between workgroups within a
// launch: the store writes through to the device coherence point, the load
// never returns a line cached before that point was updated.
__device__ __forceinline__ void st_dev(uint16_t* p, uint32_t bf_bits) {
  __hip_atomic_store(p, (uint16_t)bf_bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(float* p, float v) {
  __hip_atomic_store(p, canon(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u32x4 ld_dev16(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, AUX_SC1);
}
__device__ __forceinline__ uint32_t ld_dev4(rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, AUX_SC1);
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

// Sentinel tests. bf16 exchange data: any 16-bit lane equal to 0xffff.
// fp32 exchange data: a whole word equal to 0xffffffff.
__device__ __forceinline__ bool sent_bf16(uint32_t w) { return (w | 0xffff0000u) == 0xffffffffu || w >= 0xffff0000u; }
__device__ __forceinline__ bool sent_bf16(u32x4 v) {
  return sent_bf16(v.x) || sent_bf16(v.y) || sent_bf16(v.z) || sent_bf16(v.w);
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
  uint8_t* xch;   // exchange sets (uncached device memory)
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
// Hand-over waits: bounded polls of exchange buffers
// ---------------------------------------------------------------------------
struct Sync {
  uint32_t* err;
  unsigned long long timeout;
  unsigned long long* trace;   // this workgroup's MK_TRACE_SLOTS slots, or null
};

__device__ __forceinline__ void trace_mark(const Sync& s, int slot) {
  if (s.trace && threadIdx.x == 0 && slot < MK_TRACE_SLOTS) s.trace[slot] = wall_clock64();
}

// True when a wait must give up: its time limit passed (the error bit is set
// then) or another wait already gave up. Wave-uniform.
__device__ __forceinline__ bool wait_expired(const Sync& s, unsigned long long t0, int it) {
  if ((it & 15) == 0 &&
      (__hip_atomic_load(s.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & MK_DEVERR_SYNC))
    return true;
  if (wall_clock64() - t0 > s.timeout) {
    if (lane_id() == 0)
      __hip_atomic_fetch_or(s.err, MK_DEVERR_SYNC, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
  }
  return false;
}

// Each lane polls N 16-byte pieces of bf16 exchange data (offsets into `r`;
// OOB offsets read zero and count as ready) until the whole wave sees no
// sentinel. A piece seen complete is not read again (its offset turns OOB),
// so waiting consumers only re-read what is still missing. Called by full waves.
template <int N>
__device__ __forceinline__ void poll_bf16(const Sync& s, rsrc_t r, const uint32_t (&off)[N], u32x4 (&v)[N]) {
  const unsigned long long t0 = wall_clock64();
  bool done[N];
#pragma unroll
  for (int i = 0; i < N; ++i) done[i] = false;
  for (int it = 1;; ++it) {
    u32x4 t[N];
#pragma unroll
    for (int i = 0; i < N; ++i) t[i] = ld_dev16(r, done[i] ? OOB : off[i]);
    bool ok = true;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if (!done[i]) {
        v[i] = t[i];
        done[i] = !sent_bf16(t[i]);
      }
      ok = ok && done[i];
    }
    if (__all(ok)) return;
    if (wait_expired(s, t0, it)) return;
    __builtin_amdgcn_s_sleep(2);
  }
}

// Stage a bf16 vector of PER_WAVE*4 chunks of 512 elements into LDS: wave w
// copies chunks w, w+4, ... Exchange buffers are polled; final data (the
// embedding row, hidden_in) is read directly. The caller synchronises.
template <int PER_WAVE>
__device__ __forceinline__ void stage_vec(const Sync& s, const uint16_t* src, bool polled, uint16_t* lds) {
  const int lane = lane_id(), wave = wave_id();
  const rsrc_t r = make_rsrc(src, (size_t)PER_WAVE * NWAVE * 1024);
  uint32_t off[PER_WAVE];
  u32x4 v[PER_WAVE];
#pragma unroll
  for (int i = 0; i < PER_WAVE; ++i) off[i] = (uint32_t)((wave + NWAVE * i) * 1024 + lane * 16);
  if (polled) {
    poll_bf16<PER_WAVE>(s, r, off, v);
  } else {
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) v[i] = ld16(r, off[i]);
  }
#pragma unroll
  for (int i = 0; i < PER_WAVE; ++i) *reinterpret_cast<u32x4*>(lds + (wave + NWAVE * i) * 512 + lane * 8) = v[i];
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

// Lane slice of a 2048-vector in LDS: elements i*512 + lane*8 .. +7.
__device__ __forceinline__ void lds_x2048(const uint16_t* x, u32x4 (&xs)[4]) {
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

__device__ __forceinline__ float dot2048(const u32x4 (&wv)[4], const u32x4 (&xs)[4]) {
  float a = dot8(wv[0], xs[0], 0.f);
  float b = dot8(wv[1], xs[1], 0.f);
  a = dot8(wv[2], xs[2], a);
  b = dot8(wv[3], xs[3], b);
  return a + b;
}

// ---------------------------------------------------------------------------
// The megakernel
// ---------------------------------------------------------------------------
struct AttnShared {
  float mx[NWAVE][GQA];
  float sm[NWAVE][GQA];
  float pv[NWAVE][8][GQA * 8];
};

struct Lds {
  __attribute__((aligned(16))) uint16_t x[H];       // layer input (raw): QKV input, O residual
  __attribute__((aligned(16))) uint16_t h1[H];      // h1 (raw): GU input, DOWN residual
  __attribute__((aligned(16))) uint16_t v[INTER];   // staged GEMV input: attention output / act
  __attribute__((aligned(16))) uint16_t q[GQA * HD + 2 * HD];  // attention: 4 q heads | fresh k | fresh v
  float val[128];                                    // QKV dot products of this workgroup
  AttnShared att;
  float best[NWAVE];
  int bidx[NWAVE];
  int last;
};

struct Ctx {
  const KParams* p;
  Sync s;
  int G, w;
  int pos;
  int n_rows;            // KV rows attended: pos + 1
  const uint16_t* x_in;  // input of the first layer (embedding row or hidden_in): final data
  uint8_t* set;          // this launch's exchange buffers

  __device__ __forceinline__ uint16_t* xb(int li, size_t off) const {
    return reinterpret_cast<uint16_t*>(set + (size_t)li * X_LAYER + off);
  }
  __device__ __forceinline__ float* part(int li) const {
    return reinterpret_cast<float*>(set + (size_t)li * X_LAYER + X_PART);
  }
};

// Trace exchange index of phase `ph` (1 QKV, 2 ATTN, 3 O, 4 GU, 5 DOWN) of run-layer li.
__device__ __forceinline__ int xk(int li, int ph) { return 5 * li + ph; }

__device__ __forceinline__ u32x4 rope_pair(float a, float b, const uint16_t* rrow, int d) {
  // out[d]    = bf16(bf16(a*cos[d])    + bf16(-b*sin[d]))
  // out[d+32] = bf16(bf16(b*cos[d+32]) + bf16( a*sin[d+32]))      (attention.py:160-174)
  const float c0 = bf2f(rrow[d]), c1 = bf2f(rrow[d + 32]);
  const float s0 = bf2f(rrow[64 + d]), s1 = bf2f(rrow[64 + d + 32]);
  const float ra = rbf(rbf(a * c0) + rbf(-b * s0));
  const float rb = rbf(rbf(b * c1) + rbf(a * s1));
  return u32x4{f2bf(ra), f2bf(rb), 0u, 0u};
}

// QKV phase of run-layer li (stack layer l): RMSNorm, GEMV, RoPE; q and the
// fresh K/V row to the exchange buffer, the K/V row also into the caches.
__device__ __forceinline__ void phase_qkv(Ctx& c, int li, Lds& L) {
  const KParams& p = *c.p;
  const int l = p.first_layer + li;
  const int wave = wave_id();
  int P0, P1;
  share(QKV_PAIRS, c.G, c.w, P0, P1);
  const int nrows = 2 * (P1 - P0);
  RowStream<4, 4> rs;
  rs.start(make_rsrc(p.w_qkv + (size_t)l * QKV_ROWS * H, QKV_LAYER_BYTES),
           (uint32_t)(2 * P0 + wave) * (H * 2), NWAVE * H * 2, wave_count(0, nrows));
  trace_mark(c.s, 2 * xk(li, 1) - 1);
  if (li == 0) stage_vec<1>(c.s, c.x_in, false, L.x);
  else stage_vec<1>(c.s, c.xb(li - 1, X_H2), true, L.x);
  __syncthreads();
  trace_mark(c.s, 2 * xk(li, 1));
  u32x4 xs[4];
  lds_x2048(L.x, xs);
  rmsnorm2048(xs, nullptr);
  rs.run([&](const u32x4(&wv)[4]) { return dot2048(wv, xs); },
         [&](int r, float part) {
           const float v = wave_sum(part);
           if (lane_id() == 0) L.val[wave + NWAVE * r] = v;
         });
  __syncthreads();
  const uint16_t* rrow = p.rope + (size_t)c.pos * (2 * HD);
  uint16_t* xq = c.xb(li, X_QKV);
  for (int lp = threadIdx.x; lp < P1 - P0; lp += NT) {
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
      // the cache row is read only by later launches: a plain store
      uint16_t* crow = (is_k ? p.kc[li] : p.vc[li]) + ((size_t)kh * p.s_max + c.pos) * HD + d;
      crow[0] = (uint16_t)o.x;
      crow[32] = (uint16_t)o.y;
    }
  }
}

// One attention work item: kv head h, cached KV rows [j0, jc) plus, if
// `fresh`, the new row pos (from LDS), for the 4 q heads of the group (GQA).
// Thread t serves row (t >> 3) of each 32-row round and the 8 dims (t & 7)*8..
// of it; rows stream in groups of ATT_GROUP with an online softmax. Writes
// the item's partial (m[4], l[4], o[4][64]) unnormalised, relative to m.
__device__ __forceinline__ void attn_item(Ctx& c, int li, int h, int j0, int jc, bool fresh, float* part, Lds& L) {
  const KParams& p = *c.p;
  AttnShared& sh = L.att;
  const int t = threadIdx.x, rl = t >> 3, ch = t & 7, wave = wave_id(), lane = lane_id();
  const size_t head_bytes = (size_t)p.s_max * HD * 2;
  const rsrc_t rk = make_rsrc(p.kc[li] + (size_t)h * p.s_max * HD, head_bytes);
  const rsrc_t rv = make_rsrc(p.vc[li] + (size_t)h * p.s_max * HD, head_bytes);
  u32x4 q[GQA];
#pragma unroll
  for (int g = 0; g < GQA; ++g) q[g] = *reinterpret_cast<const u32x4*>(L.q + g * HD + ch * 8);
  float m_run[GQA], l_run[GQA], acc[GQA][8];
#pragma unroll
  for (int g = 0; g < GQA; ++g) {
    m_run[g] = -INFINITY;
    l_run[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  }
  constexpr int R = ATT_GROUP / 32;
  auto consume = [&](const u32x4(&kk)[R], const u32x4(&vv)[R], const bool(&valid)[R]) {
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
  };
  for (int base = j0; base < jc; base += ATT_GROUP) {
    u32x4 kk[R], vv[R];
    bool valid[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int j = base + 32 * r + rl;
      valid[r] = j < jc;
      const uint32_t off = valid[r] ? (uint32_t)(j * HD + ch * 8) * 2u : OOB;
      kk[r] = ld_stream(rk, off);
      vv[r] = ld_stream(rv, off);
    }
    consume(kk, vv, valid);
  }
  if (fresh) {   // the new row: row-lane 0 of the first round
    u32x4 kk[R], vv[R];
    bool valid[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      valid[r] = r == 0 && rl == 0;
      kk[r] = valid[r] ? *reinterpret_cast<const u32x4*>(L.q + GQA * HD + ch * 8) : u32x4{0u, 0u, 0u, 0u};
      vv[r] = valid[r] ? *reinterpret_cast<const u32x4*>(L.q + GQA * HD + HD + ch * 8) : u32x4{0u, 0u, 0u, 0u};
    }
    consume(kk, vv, valid);
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

// Merge the nsplit partials of kv head h (polled) into the bf16 attention
// output of its 4 q heads:
//   att = sum_s e^(m_s-M) o_s / sum_s e^(m_s-M) l_s   (then cast to bf16)
// Thread t produces q head 4h + (t >> 6), dim t & 63.
__device__ __forceinline__ void attn_merge_head(Ctx& c, int li, int h, int nsplit) {
  const int t = threadIdx.x, g = t >> 6, d = t & 63;
  const rsrc_t r = make_rsrc(c.part(li) + (size_t)h * ATT_MAX_SPLIT * PART_FLOATS,
                             (size_t)nsplit * PART_FLOATS * 4);
  uint32_t m[ATT_MAX_SPLIT], l[ATT_MAX_SPLIT], o[ATT_MAX_SPLIT];
  const unsigned long long t0 = wall_clock64();
  for (int it = 1;; ++it) {
    bool ok = true;
#pragma unroll
    for (int s = 0; s < ATT_MAX_SPLIT; ++s) {   // splits >= nsplit read zero (out of range)
      const uint32_t base = (uint32_t)(s * PART_FLOATS) * 4u;
      m[s] = ld_dev4(r, base + (uint32_t)g * 4u);
      l[s] = ld_dev4(r, base + (uint32_t)(GQA + g) * 4u);
      o[s] = ld_dev4(r, base + (uint32_t)(2 * GQA + g * HD + d) * 4u);
    }
#pragma unroll
    for (int s = 0; s < ATT_MAX_SPLIT; ++s) ok = ok && m[s] != 0xffffffffu && l[s] != 0xffffffffu && o[s] != 0xffffffffu;
    if (__all(ok)) break;
    if (wait_expired(c.s, t0, it)) break;
    __builtin_amdgcn_s_sleep(1);
  }
  float M = -INFINITY;
#pragma unroll
  for (int s = 0; s < ATT_MAX_SPLIT; ++s)
    if (s < nsplit) M = fmaxf(M, __uint_as_float(m[s]));
  float O = 0.f, Lsum = 0.f;
#pragma unroll
  for (int s = 0; s < ATT_MAX_SPLIT; ++s) {
    const float wgt = s < nsplit ? __expf(__uint_as_float(m[s]) - M) : 0.f;
    Lsum = fmaf(wgt, __uint_as_float(l[s]), Lsum);
    O = fmaf(wgt, __uint_as_float(o[s]), O);
  }
  const uint32_t mine = f2bf(O / Lsum);
  const uint32_t next = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mine, DPP_XOR1, 0xf, 0xf, false);
  if ((d & 1) == 0)
    st_dev(reinterpret_cast<uint32_t*>(c.xb(li, X_ATT) + (h * GQA + g) * HD + d), mine | (next << 16));
}

// ATTN phase: the workgroup's attention items (kv head, KV split).
__device__ __forceinline__ void phase_attn(Ctx& c, int li, Lds& L) {
  int nsplit, rows;
  attn_split(c.n_rows, nsplit, rows);
  const int nitems = NKV * nsplit;
  const int lane = lane_id();
  for (int it = c.w; it < nitems; it += c.G) {
    const int h = it / nsplit, sp = it % nsplit;
    const int j0 = sp * rows, j1 = min(j0 + rows, c.n_rows);
    const bool fresh = c.pos >= j0 && c.pos < j1;
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
    __syncthreads();
    if (it == c.w) trace_mark(c.s, 2 * xk(li, 2));
    attn_item(c, li, h, j0, min(j1, c.pos), fresh,
              c.part(li) + ((size_t)h * ATT_MAX_SPLIT + sp) * PART_FLOATS, L);
    if (sp == 0) attn_merge_head(c, li, h, nsplit);
  }
}

__global__ void __launch_bounds__(NT, 1) mk_decode_kernel(KParams p) {
  __shared__ Lds L;

  Ctx c;
  c.p = &p;
  uint32_t* ctrl = reinterpret_cast<uint32_t*>(p.ws);
  c.s.err = ctrl + C_ERR;
  c.s.timeout = p.timeout_ticks;
  c.s.trace = p.trace ? p.trace + (size_t)blockIdx.x * MK_TRACE_SLOTS : nullptr;
  trace_mark(c.s, 0);
  c.G = gridDim.x;
  c.w = blockIdx.x;
  const uint32_t epoch = __hip_atomic_load(ctrl + C_EPOCH, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  c.set = p.xch + (size_t)(epoch & 1u) * SET_BYTES;
  {
    // refill the other set with the sentinel for the next launch
    u32x4* other = reinterpret_cast<u32x4*>(p.xch + (size_t)((epoch + 1u) & 1u) * SET_BYTES);
    const size_t n = SET_BYTES / 16;
    int lo, hi;
    share((int)n, c.G, c.w, lo, hi);
    for (int i = lo + threadIdx.x; i < hi; i += NT) other[i] = u32x4{~0u, ~0u, ~0u, ~0u};
  }
  c.pos = p.pos[0];
  const bool pos_ok = c.pos >= 0 && c.pos < p.s_max && c.pos < p.rope_rows;
  if (!pos_ok && blockIdx.x == 0 && threadIdx.x == 0)
    __hip_atomic_fetch_or(c.s.err, MK_DEVERR_POS, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  c.n_rows = c.pos + 1;
  if (p.hidden_in) {
    c.x_in = p.hidden_in;
  } else {
    int tok = p.tokens[0];
    tok = tok < 0 ? 0 : (tok >= VOCAB ? VOCAB - 1 : tok);
    c.x_in = p.embed + (size_t)tok * H;
  }
  const int G = c.G, w = c.w, wave = wave_id(), lane = lane_id();

  if (pos_ok) {
    int R0, R1;
    share(H, G, w, R0, R1);
    for (int li = 0; li < p.n_layers; ++li) {
      const int l = p.first_layer + li;
      const bool last = li == p.n_layers - 1;
      phase_qkv(c, li, L);
      phase_attn(c, li, L);

      // ---- O projection + residual -> h1 ----
      {
        RowStream<2, 4> os;
        const Span sp = wave_span(R0, R1);
        os.start(make_rsrc(p.w_o + (size_t)l * H * H, O_LAYER_BYTES), (uint32_t)sp.lo * (H * 2), H * 2, sp.n);
        trace_mark(c.s, 2 * xk(li, 3) - 1);
        stage_vec<1>(c.s, c.xb(li, X_ATT), true, L.v);
        __syncthreads();
        trace_mark(c.s, 2 * xk(li, 3));
        u32x4 xs[4];
        lds_x2048(L.v, xs);
        uint16_t* h1 = c.xb(li, X_H1);
        float mine = 0.f;   // lane r: the wave's row r
        os.run([&](const u32x4(&wv)[4]) { return dot2048(wv, xs); },
               [&](int r, float part) {
                 const float v = wave_sum(part);
                 if (lane == r) mine = v;
               });
        if (lane < sp.n) st_dev(h1 + sp.lo + lane, f2bf(bf2f(L.x[sp.lo + lane]) + rbf(mine)));
      }

      // ---- gate/up + SwiGLU -> act ----
      {
        int U0, U1;
        share(INTER, G, w, U0, U1);
        RowStream<4, 8> gs;
        const Span sp = wave_span(U0, U1);
        gs.start(make_rsrc(p.w_gu + (size_t)l * 2 * INTER * H, GU_LAYER_BYTES), (uint32_t)sp.lo * (2 * H * 2),
                 2 * H * 2, sp.n);
        trace_mark(c.s, 2 * xk(li, 4) - 1);
        stage_vec<1>(c.s, c.xb(li, X_H1), true, L.h1);
        __syncthreads();
        trace_mark(c.s, 2 * xk(li, 4));
        u32x4 xs[4];
        lds_x2048(L.h1, xs);
        rmsnorm2048(xs, nullptr);
        uint16_t* act = c.xb(li, X_ACT);
        struct GU2 { float g, u; };
        float mine = 0.f;   // lane r: silu(gate) * up of the wave's pair r
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
                 if (lane == r) mine = gv / (1.0f + __expf(-gv)) * uv;
               });
        if (lane < sp.n) st_dev(act + sp.lo + lane, f2bf(mine));
      }

      // ---- down projection + residual -> h2 ----
      {
        RowStream<2, 16> ds;
        const Span sp = wave_span(R0, R1);
        ds.start(make_rsrc(p.w_d + (size_t)l * H * INTER, D_LAYER_BYTES), (uint32_t)sp.lo * (INTER * 2), INTER * 2,
                 sp.n);
        trace_mark(c.s, 2 * xk(li, 5) - 1);
        stage_vec<4>(c.s, c.xb(li, X_ACT), true, L.v);
        __syncthreads();
        trace_mark(c.s, 2 * xk(li, 5));
        uint16_t* h2 = c.xb(li, X_H2);
        u32x4 xs[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) xs[i] = *reinterpret_cast<const u32x4*>(L.v + i * 512 + lane * 8);
        float mine = 0.f;   // lane r: the wave's row r
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
                 if (lane == r) mine = v;
               });
        if (lane < sp.n) {
          const int row = sp.lo + lane;
          const uint32_t hv = f2bf(bf2f(L.h1[row]) + rbf(mine));
          st_dev(h2 + row, hv);
          if (last && p.hidden_out) p.hidden_out[row] = (uint16_t)hv;
        }
      }
    }

    // ---- final norm + tied lm_head + argmax ----
    if (p.do_lm) {
      int V0, V1;
      share(VOCAB, G, w, V0, V1);
      RowStream<8, 4> ls;
      const Span sp = wave_span(V0, V1);
      ls.start(make_rsrc(p.embed, EMBED_BYTES), (uint32_t)sp.lo * (H * 2), H * 2, sp.n);
      trace_mark(c.s, 2 * xk(p.n_layers, 1) - 1);
      stage_vec<1>(c.s, c.xb(p.n_layers - 1, X_H2), true, L.x);
      __syncthreads();
      trace_mark(c.s, 2 * xk(p.n_layers, 1));
      u32x4 xs[4];
      lds_x2048(L.x, xs);
      rmsnorm2048(xs, p.g_final);
      float best = -INFINITY;
      int bidx = 0x7fffffff;
      ls.run([&](const u32x4(&wv)[4]) { return dot2048(wv, xs); },
             [&](int r, float part) {
               const float v = wave_sum(part);
               const int row = sp.lo + r;
               if (lane == 0 && p.logits) p.logits[row] = v;
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
      if (threadIdx.x == 0) {
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
          __hip_atomic_fetch_max(reinterpret_cast<unsigned long long*>(p.ws + C_KEY_BYTE), key,
                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
  }

  // ---- exit: the last workgroup out publishes the token and advances the epoch ----
  trace_mark(c.s, MK_TRACE_SLOTS - 1);
  wait_mem();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(ctrl + C_EXIT, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    L.last = prev == (uint32_t)(G - 1);
  }
  __syncthreads();
  if (!L.last || threadIdx.x != 0) return;
  ctrl[C_EXIT] = 0u;
  ctrl[C_EPOCH] = epoch + 1u;
  if (pos_ok) {
    if (p.do_lm) {
      unsigned long long* kp = reinterpret_cast<unsigned long long*>(p.ws + C_KEY_BYTE);
      const unsigned long long key = __hip_atomic_load(kp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *kp = 0ull;
      if (p.next_token) p.next_token[0] = (int32_t)(0xffffffffu - (uint32_t)(key & 0xffffffffull));
    }
    if (p.flags & MK_FLAG_ADVANCE) p.pos[0] = c.pos + 1;
  }
}

// Fill kernel: the first n_zero 16-byte units zeroed (the control block), the
// rest set to the exchange sentinel (all ones).
__global__ void mk_ws_init_kernel(u32x4* p, size_t n, size_t n_zero) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = i < n_zero ? u32x4{0u, 0u, 0u, 0u} : u32x4{~0u, ~0u, ~0u, ~0u};
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

// Exchange areas. The per-layer hand-over buffers live in uncached device
// memory: with it an all-to-all hand-over under a full HBM weight stream took
// 3.8 us against 6 us in ordinary (L2-cached) memory. Each workspace gets one
// area of XCH_BYTES, created by its first mk_workspace_init on a device and
// kept until the process ends: uncached memory that a kernel has read must
// not be freed while the process runs.
constexpr size_t XCH_BYTES = 2 * SET_BYTES;
struct XchEntry {
  const void* ws;
  int dev;
  uint8_t* xch;
};
XchEntry g_xch[256];
int g_n_xch = 0;
std::mutex g_xch_mu;

uint8_t* exchange_of(const void* ws, int dev) {
  std::lock_guard<std::mutex> lk(g_xch_mu);
  for (int i = 0; i < g_n_xch; ++i)
    if (g_xch[i].ws == ws && g_xch[i].dev == dev) return g_xch[i].xch;
  return nullptr;
}

int exchange_create(const void* ws, int dev, uint8_t** out) {
  std::lock_guard<std::mutex> lk(g_xch_mu);
  for (int i = 0; i < g_n_xch; ++i)
    if (g_xch[i].ws == ws && g_xch[i].dev == dev) {
      *out = g_xch[i].xch;
      return MK_OK;
    }
  if (g_n_xch == (int)(sizeof(g_xch) / sizeof(g_xch[0])))
    return fail(MK_ERR_WORKSPACE, "too many workspaces initialised in this process (%d)", g_n_xch);
  void* p = nullptr;
  const hipError_t e = hipExtMallocWithFlags(&p, XCH_BYTES, hipDeviceMallocUncached);
  if (e != hipSuccess) return fail(MK_ERR_HIP, "exchange area allocation: %s", hipGetErrorString(e));
  g_xch[g_n_xch++] = XchEntry{ws, dev, static_cast<uint8_t*>(p)};
  *out = static_cast<uint8_t*>(p);
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
  if (workspace_bytes < WS_BYTES)
    return fail(MK_ERR_WORKSPACE, "workspace %zu bytes < %zu needed", workspace_bytes, WS_BYTES);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(MK_ERR_HIP, "hipGetDevice failed");
  uint8_t* xch = nullptr;
  int rc = exchange_create(workspace, dev, &xch);
  if (rc != MK_OK) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t n = workspace_bytes / 16;
  hipLaunchKernelGGL(mk_ws_init_kernel, dim3((int)((n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024)), dim3(256), 0,
                     st, static_cast<u32x4*>(workspace), n, n);
  hipLaunchKernelGGL(mk_ws_init_kernel, dim3(1024), dim3(256), 0, st, reinterpret_cast<u32x4*>(xch),
                     XCH_BYTES / 16, (size_t)0);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MK_ERR_HIP, "workspace init launch: %s", hipGetErrorString(e));
  return MK_OK;
}

int mk_read_device_error(void* workspace, void* stream, uint32_t* bits_out) {
  if (!workspace || !bits_out) return fail(MK_ERR_NULL, "workspace or bits_out is NULL");
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e = hipStreamSynchronize(st);
  if (e != hipSuccess) return fail(MK_ERR_HIP, "hipStreamSynchronize: %s", hipGetErrorString(e));
  uint32_t* dev_err = reinterpret_cast<uint32_t*>(workspace) + C_ERR;
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
  uint8_t* xch = exchange_of(a->workspace, dev);
  if (!xch) return fail(MK_ERR_WORKSPACE, "workspace was not initialised with mk_workspace_init on device %d", dev);

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
  kp.xch = xch;
  kp.first_layer = a->first_layer;
  kp.n_layers = a->n_layers;
  kp.s_max = a->s_max;
  kp.rope_rows = w->rope_rows;
  kp.do_lm = do_lm ? 1 : 0;
  kp.flags = a->flags;
  kp.timeout_ticks = di.ticks_per_s * 2ull;   // 2 s per hand-over wait
  kp.trace = static_cast<unsigned long long*>(a->trace);

  void* args[] = {&kp};
  // One workgroup per CU with occupancy 1 (checked in device_info): on an
  // otherwise idle device a plain launch makes every workgroup resident at
  // once, and leaves ~20 us less between consecutive steps than a cooperative
  // launch. MK_FLAG_COOPERATIVE asks for the guarantee. Every wait in the
  // kernel is bounded, so a workgroup that is never scheduled shows up as
  // MK_DEVERR_SYNC, not as a hang.
  const hipStream_t st = static_cast<hipStream_t>(a->stream);
  const hipError_t e =
      (a->flags & MK_FLAG_COOPERATIVE)
          ? hipLaunchCooperativeKernel(reinterpret_cast<const void*>(mk_decode_kernel), dim3(di.grid), dim3(NT), args,
                                       0, st)
          : hipLaunchKernel(reinterpret_cast<const void*>(mk_decode_kernel), dim3(di.grid), dim3(NT), args, 0, st);
  if (e != hipSuccess) return fail(MK_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e));
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
