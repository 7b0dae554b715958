// mk_common.h — device building blocks shared by the decode kernels of
// libmk.so (mk_decode.hip: batch 1; mk_batch.hip: batches of 2..32).
//
// Numerics follow the reference's NKI kernels (nki_kernels/attention.py,
// nki_kernels/mlp.py): bf16 storage, fp32 accumulation, bf16 rounding at the
// same points. Hand-over waits poll sentinel-filled exchange buffers (see the
// kernels' headers).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mk.h"

namespace mk {

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
constexpr int ATT_GROUP = 128;             // KV rows an attention item loads at once (4 rounds of 32)
constexpr int PART_FLOATS = GQA * (HD + 2);  // per split: m[4], l[4], o[4][64]
constexpr uint32_t OOB = 0x80000000u;      // buffer offset past every resource
constexpr float EPS = 1e-5f;
constexpr float SM_SCALE = 0.125f;         // 1/sqrt(64)

// The thread's index in its workgroup. tid_opaque() reads it through an
// empty volatile asm, so the compiler can neither hoist arithmetic on it out
// of a loop nor merge two reads: values such as per-lane offsets and LDS
// addresses are then recomputed where they are used instead of being kept in
// registers across the layer loop. Whether that pays depends on the kernel
// (it frees registers, and each read is a point the scheduler does not move
// memory operations across): a translation unit that defines MK_OPAQUE_TID
// before including this header gets it at every tid() use.
__device__ __forceinline__ unsigned tid_opaque() {
  unsigned v = __builtin_amdgcn_workitem_id_x();
  asm volatile("" : "+v"(v));
  return v;
}
__device__ __forceinline__ unsigned tid() {
#ifdef MK_OPAQUE_TID
  return tid_opaque();
#else
  return threadIdx.x;
#endif
}

constexpr size_t QKV_LAYER_BYTES = (size_t)QKV_ROWS * H * 2;
constexpr size_t O_LAYER_BYTES = (size_t)H * H * 2;
constexpr size_t GU_LAYER_BYTES = (size_t)2 * INTER * H * 2;
constexpr size_t D_LAYER_BYTES = (size_t)H * INTER * 2;
constexpr size_t EMBED_BYTES = (size_t)VOCAB * H * 2;

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
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) { return f2bf(lo) | (f2bf(hi) << 16); }
// Two floats -> packed bf16x2 with the hardware conversion (v_cvt_pk_bf16_f32,
// round to nearest even, equal to f2bf bit for bit except that a NaN keeps
// its payload, so it may be 0xffff): for values that stay in registers.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t cvt_bf2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));
}
// fp32 rounded to bf16 precision (hardware conversion; registers only).
__device__ __forceinline__ float rbf(float f) { return __uint_as_float(cvt_bf2(f, 0.f) << 16); }
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

constexpr int DPP_HALF_MIRROR = 0x141;  // row_half_mirror: lane i of each 8-lane group reads lane 7-i

// Sum over each aligned group of 8 lanes (8k .. 8k+7), in every lane of the
// group: after the two quad steps both quads of the group are uniform, so the
// half-row mirror adds the other quad (the same sums as xor-4 butterflies).
__device__ __forceinline__ float sum_lanes8(float v) {
  v += dpp<DPP_XOR1>(v);
  v += dpp<DPP_XOR2>(v);
  return v + dpp<DPP_HALF_MIRROR>(v);
}

// Lane i's value and lane i^16 / i^32's (gfx950 permlane swaps). The swap
// exchanges the odd 16-lane rows of its first register with the even rows of
// its second (or the upper 32 lanes of the first with the lower 32 of the
// second); with both registers holding v it leaves
// {v of rows 0,0,2,2 | rows 1,1,3,3} or {v of lanes 0-31 twice | 32-63 twice}.
// Inline assembly: both registers are read and written, which the compiler's
// builtin for these instructions does not model here (it aliases the two
// results). The s_nops cover the VALU-write -> permlane-read hazard.
struct Pair {
  float a, b;
};
__device__ __forceinline__ Pair xor16_pair(float v) {
  float a = v, b = v;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return Pair{a, b};
}
__device__ __forceinline__ Pair xor32_pair(float v) {
  float a = v, b = v;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return Pair{a, b};
}
__device__ __forceinline__ float add_xor16(float v) {
  const Pair p = xor16_pair(v);
  return p.a + p.b;
}
__device__ __forceinline__ float add_xor32(float v) {
  const Pair p = xor32_pair(v);
  return p.a + p.b;
}
__device__ __forceinline__ float max_xor16(float v) {
  const Pair p = xor16_pair(v);
  return fmaxf(p.a, p.b);
}
__device__ __forceinline__ float max_xor32(float v) {
  const Pair p = xor32_pair(v);
  return fmaxf(p.a, p.b);
}
// Sum / max over the 8 lanes of the wave with the same lane & 7 (lane ^ 8, ^16, ^32).
__device__ __forceinline__ float sum_stride8(float v) {
  v += dpp<DPP_ROR8>(v);   // within a 16-lane row, lane i^8
  return add_xor32(add_xor16(v));
}
__device__ __forceinline__ float max_stride8(float v) {
  v = fmaxf(v, dpp<DPP_ROR8>(v));
  return max_xor32(max_xor16(v));
}

// Transposed reduction of N = 1, 2, 4, 8 or 16 per-lane partial sums (one per
// GEMV row) over the 64 lanes: one exchange step per lane bit halves both the
// values per lane and the lanes per row, so N rows cost about 2N + 8
// instructions instead of N full wave sums. Returns, in lane i, the full sum
// of row reduce_row<N>(i); each row's sum is held by 64/N lanes.
//   bit 5: permlane32 swap of rows (k, k+N/2)   bit 4: permlane16 swap
//   bit 3: DPP row_ror:8 (lane ^ 8)             bit 2: DPP row_half_mirror (lane ^ 7)
// at each step the lanes with the bit clear keep the lower row of the pair.
// The remaining lane bits are then summed with plain steps (quads first).
template <int N>
__device__ __forceinline__ int reduce_row(int lane) {
  static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16, "N rows per reduction");
  int r = 0, w = N;
  if (w > 1) { w >>= 1; r += ((lane >> 5) & 1) * w; }
  if (w > 1) { w >>= 1; r += ((lane >> 4) & 1) * w; }
  if (w > 1) { w >>= 1; r += ((lane >> 3) & 1) * w; }
  if (w > 1) { w >>= 1; r += ((lane >> 2) & 1) * w; }
  return r;
}
__device__ __forceinline__ Pair swap32(float a, float b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return Pair{a, b};
}
__device__ __forceinline__ Pair swap16(float a, float b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return Pair{a, b};
}
template <int N>
__device__ __forceinline__ float reduce_rows(const float (&in)[N]) {
  const int lane = tid() & 63;
  float v[N];
#pragma unroll
  for (int k = 0; k < N; ++k) v[k] = in[k];
  int n = N;
  // bit 5: lanes 0-31 end up with rows k, lanes 32-63 with rows k + n/2
  if (n > 1) {
    n >>= 1;
#pragma unroll
    for (int k = 0; k < N / 2; ++k) {
      const Pair p = swap32(v[k], v[k + N / 2]);
      v[k] = p.a + p.b;
    }
  } else {
    v[0] = add_xor32(v[0]);
  }
  // bit 4
  if (n > 1) {
    n >>= 1;
#pragma unroll
    for (int k = 0; k < N / 4; ++k) {
      const Pair p = swap16(v[k], v[k + N / 4]);
      v[k] = p.a + p.b;
    }
  } else {
    v[0] = add_xor16(v[0]);
  }
  // bit 3 (lane ^ 8 within a 16-lane row)
  const bool b3 = lane & 8, b2 = lane & 4;
  if (n > 1) {
    n >>= 1;
#pragma unroll
    for (int k = 0; k < N / 8; ++k) {
      const float keep = b3 ? v[k + N / 8] : v[k], give = b3 ? v[k] : v[k + N / 8];
      v[k] = keep + dpp<DPP_ROR8>(give);
    }
  }
  // bit 2 (lane ^ 7 within an 8-lane group)
  if (n > 1) {
    n >>= 1;
#pragma unroll
    for (int k = 0; k < N / 16; ++k) {
      const float keep = b2 ? v[k + N / 16] : v[k], give = b2 ? v[k] : v[k + N / 16];
      v[k] = keep + dpp<DPP_HALF_MIRROR>(give);
    }
  }
  // plain sums over the lane bits not used above: quads, then the rest
  float x = v[0];
  x += dpp<DPP_XOR1>(x);
  x += dpp<DPP_XOR2>(x);
  if (N < 16) x += dpp<DPP_HALF_MIRROR>(x);
  if (N < 8) x += dpp<DPP_ROR8>(x);
  return x;
}

// In-place sum (or max) of N = 4 or 32 per-lane values over the 8 lanes that
// share lane & 7 (lane bits 3-5), transposed like reduce_rows: afterwards
// v[0 .. N/8) of lane i hold values (4*b5 + 2*b4 + b3) * N/8 + k of the
// original array (for N = 4: v[0] holds value 2*b5 + b4).
template <int N, bool MAX>
__device__ __forceinline__ void reduce_stride8(float (&v)[N]) {
  static_assert(N == 4 || N == 32, "4 or 32 values");
  const int lane = tid() & 63;
  auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
#pragma unroll
  for (int k = 0; k < N / 2; ++k) {
    const Pair p = swap32(v[k], v[k + N / 2]);
    v[k] = op(p.a, p.b);
  }
#pragma unroll
  for (int k = 0; k < N / 4; ++k) {
    const Pair p = swap16(v[k], v[k + N / 4]);
    v[k] = op(p.a, p.b);
  }
  if (N == 4) {
    v[0] = op(v[0], dpp<DPP_ROR8>(v[0]));
  } else {
    const bool b3 = lane & 8;
#pragma unroll
    for (int k = 0; k < N / 8; ++k) {
      const float keep = b3 ? v[k + N / 8] : v[k], give = b3 ? v[k] : v[k + N / 8];
      v[k] = op(keep, dpp<DPP_ROR8>(give));
    }
  }
}

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
// (The builtin, not inline assembly: the compiler's own wait insertion then
// knows that nothing issued before it is still outstanding.)
__device__ __forceinline__ void wait_mem() { __builtin_amdgcn_s_waitcnt(0x0f70); }   // vmcnt(0)

// Workgroup barrier for data exchanged through LDS by ds_write / ds_read.
// __syncthreads() (and an LDS-only fence, once a wave has HBM -> LDS copies in
// flight) also waits for every outstanding global load and store of the wave
// (s_waitcnt vmcnt(0)), which holds the barrier back until weight streams and
// background copies issued before it have landed; this one leaves them in
// flight. A wave reads an LDS area written by its own HBM -> LDS copies only
// after wait_mem().
__device__ __forceinline__ void lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ int lane_id() { return tid() & 63; }
__device__ __forceinline__ int wave_id() { return tid() >> 6; }

// Contiguous share [lo, hi) of `total` items for part `i` of `n`.
// (32-bit division when the products fit: much shorter than the 64-bit one.)
__device__ __forceinline__ void share(int total, int n, int i, int& lo, int& hi) {
  if ((unsigned long long)(unsigned)total * (unsigned)n <= 0xffffffffull) {
    lo = (int)(((uint32_t)total * (uint32_t)i) / (uint32_t)n);
    hi = (int)(((uint32_t)total * (uint32_t)(i + 1)) / (uint32_t)n);
  } else {
    lo = (int)(((long long)total * i) / n);
    hi = (int)(((long long)total * (i + 1)) / n);
  }
}

// Sentinel tests. bf16 exchange data: any 16-bit lane equal to 0xffff.
// fp32 exchange data: a whole word equal to 0xffffffff.
__device__ __forceinline__ bool sent_bf16(uint32_t w) { return (w | 0xffff0000u) == 0xffffffffu || w >= 0xffff0000u; }
__device__ __forceinline__ bool sent_bf16(u32x4 v) {
  return sent_bf16(v.x) || sent_bf16(v.y) || sent_bf16(v.z) || sent_bf16(v.w);
}

// ---------------------------------------------------------------------------
// Hand-over waits: bounded polls of exchange buffers
// ---------------------------------------------------------------------------
struct Sync {
  uint32_t* err;
  unsigned long long timeout;
  unsigned long long* trace;   // this workgroup's MK_TRACE_SLOTS slots, or null
};

__device__ __forceinline__ void trace_mark(const Sync& s, int slot) {
  if (s.trace && tid() == 0 && slot < MK_TRACE_SLOTS) s.trace[slot] = wall_clock64();
}
// Slot MK_TRACE_DONE0 + 5*li + j: phase j (0 QKV, 1 ATTN, 2 O, 3 GU, 4 DOWN) of
// run-layer li has issued its result stores.
__device__ __forceinline__ void trace_done(const Sync& s, int li, int j) {
  if (MK_TRACE_DONE0 + 5 * li + j < MK_TRACE_SLOTS - 8) trace_mark(s, MK_TRACE_DONE0 + 5 * li + j);
}
// A diagnostic value (not a time) in one of the slots MK_TRACE_SLOTS-8 .. -2.
__device__ __forceinline__ void trace_value(const Sync& s, int k, unsigned long long v) {
  if (s.trace && tid() == 0 && k >= 0 && k < 7) s.trace[MK_TRACE_SLOTS - 8 + k] = v;
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
// idle() runs right after each round's poll loads are issued: a caller issues
// background loads there. Loads complete in order, so a background load issued
// before a poll would hold the poll's result back until it lands; issued after
// it, and in a fixed number (so the wait can count past them), it does not.
struct NoIdle {
  __device__ __forceinline__ void operator()() const {}
};
template <int N, class Idle = NoIdle>
__device__ __forceinline__ void poll_bf16(const Sync& s, rsrc_t r, const uint32_t (&off)[N], u32x4 (&v)[N],
                                          Idle&& idle = Idle()) {
  const unsigned long long t0 = wall_clock64();
  bool done[N];
#pragma unroll
  for (int i = 0; i < N; ++i) done[i] = false;
  for (int it = 1;; ++it) {
    u32x4 t[N];
#pragma unroll
    for (int i = 0; i < N; ++i) t[i] = ld_dev16(r, done[i] ? OOB : off[i]);
    idle();
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
template <int PER_WAVE, class Idle = NoIdle>
__device__ __forceinline__ void stage_vec(const Sync& s, const uint16_t* src, bool polled, uint16_t* lds,
                                          Idle&& idle = Idle()) {
  const int lane = lane_id(), wave = wave_id();
  const rsrc_t r = make_rsrc(src, (size_t)PER_WAVE * NWAVE * 1024);
  uint32_t off[PER_WAVE];
  u32x4 v[PER_WAVE];
#pragma unroll
  for (int i = 0; i < PER_WAVE; ++i) off[i] = (uint32_t)((wave + NWAVE * i) * 1024 + lane * 16);
  if (polled) {
    poll_bf16<PER_WAVE>(s, r, off, v, idle);
  } else {
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) v[i] = ld16(r, off[i]);
  }
#pragma unroll
  for (int i = 0; i < PER_WAVE; ++i) *reinterpret_cast<u32x4*>(lds + (wave + NWAVE * i) * 512 + lane * 8) = v[i];
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
      const uint32_t n = cvt_bf2(bf_lo(w[j]) * inv, bf_hi(w[j]) * inv);
      w[j] = gamma ? cvt_bf2(bf_lo(g[j]) * bf_lo(n), bf_hi(g[j]) * bf_hi(n)) : n;
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

// Element offset of (row m, column j) in a bf16 matrix kept in MFMA A-tile
// order with kblocks = columns / 32: the 1 KiB block (m / 16, j / 32), 16-byte
// slot ((j % 32) / 8) * 16 + m % 16 (the lane of v_mfma_f32_16x16x32_bf16 that
// takes it), element j % 8.
__device__ __forceinline__ size_t a_tile_off(int m, int j, int kblocks) {
  return ((size_t)(m >> 4) * (size_t)kblocks + (size_t)(j >> 5)) * 512 +
         (size_t)((((j & 31) >> 3) << 4) + (m & 15)) * 8 + (size_t)(j & 7);
}

struct AttnShared {
  float mx[NWAVE][GQA];
  float sm[NWAVE][GQA];
  float pv[NWAVE][8][GQA * 8];
};

// rrow: the position's row of the RoPE table, bf16 cos[64] | sin[64].
__device__ __forceinline__ u32x4 rope_pair(float a, float b, const uint16_t* rrow, int d) {
  // out[d]    = bf16(bf16(a*cos[d])    + bf16(-b*sin[d]))
  // out[d+32] = bf16(bf16(b*cos[d+32]) + bf16( a*sin[d+32]))      (attention.py:160-174)
  const float c0 = bf2f(rrow[d]), c1 = bf2f(rrow[d + 32]);
  const float s0 = bf2f(rrow[64 + d]), s1 = bf2f(rrow[64 + d + 32]);
  const float ra = rbf(rbf(a * c0) + rbf(-b * s0));
  const float rb = rbf(rbf(b * c1) + rbf(a * s1));
  return u32x4{f2bf(ra), f2bf(rb), 0u, 0u};
}


template <bool V>
struct BoolC {
  static constexpr bool value = V;
};

// K/V rows of an attention item streamed a group of R rounds of 32 rows at a
// time (ATT_GROUP rows by default): thread t loads row (t >> 3) of each round,
// dims (t & 7)*8 .. +7, of K and of V. Rows >= jc read zero through OOB
// offsets and are flagged invalid.
constexpr int ATT_R = ATT_GROUP / 32;
template <int R = ATT_R>
struct AttnGroupT {
  u32x4 k[R], v[R];
  bool valid[R];
};
struct AttnRows {
  rsrc_t rk, rv;
  int j0, jc;
  __device__ __forceinline__ void init(const uint16_t* kc_head, const uint16_t* vc_head, int s_max, int j0_,
                                       int jc_) {
    const size_t head_bytes = (size_t)s_max * HD * 2;
    rk = make_rsrc(kc_head, head_bytes);
    rv = make_rsrc(vc_head, head_bytes);
    j0 = j0_;
    jc = jc_;
  }
  template <int R>
  __device__ __forceinline__ int ngroups() const { return jc > j0 ? (jc - j0 + 32 * R - 1) / (32 * R) : 0; }
  template <int R>
  __device__ __forceinline__ void load(int gi, AttnGroupT<R>& g) const {
    const int rl = tid() >> 3, ch = tid() & 7;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int j = j0 + gi * 32 * R + 32 * r + rl;
      g.valid[r] = j < jc;
      const uint32_t off = g.valid[r] ? (uint32_t)(j * HD + ch * 8) * 2u : OOB;
      g.k[r] = ld_stream(rk, off);
      g.v[r] = ld_stream(rv, off);
    }
  }
};

// One attention work item: one kv head of one sequence, cached KV rows
// [j0, jc) plus, if `fresh`, the new row (from LDS), for the 4 q heads of the
// group (GQA). `rows` describes the head's cache rows (bf16 [s_max][64] for K
// and for V); `first` holds its first group, already issued with rows.load(0)
// (the cached rows do not depend on the current step, so a caller issues them
// before it waits for q). q_lds: bf16 q[4][64] | fresh k[64] | fresh v[64] in LDS.
// Thread t serves row (t >> 3) of each 32-row round and the 8 dims (t & 7)*8..
// of it; rows stream in groups of ATT_GROUP with an online softmax, the next
// group in flight. Writes the item's partial (m[4], l[4], o[4][64])
// unnormalised, relative to m.
template <int R = ATT_R>
__device__ __forceinline__ void attn_item(const AttnRows& rows, AttnGroupT<R>& first, const uint16_t* q_lds,
                                          bool fresh, float* part, AttnShared& sh) {
  const int t = tid(), rl = t >> 3, ch = t & 7, wave = wave_id(), lane = lane_id();
  u32x4 q[GQA];
#pragma unroll
  for (int g = 0; g < GQA; ++g) q[g] = *reinterpret_cast<const u32x4*>(q_lds + g * HD + ch * 8);
  float m_run[GQA], l_run[GQA], acc[GQA][8];
#pragma unroll
  for (int g = 0; g < GQA; ++g) {
    m_run[g] = -INFINITY;
    l_run[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  }
  // consume rounds of 32 rows (RA = rounds in the arrays, the first nr of them
  // holding any valid row): online softmax update
  auto consume = [&](const auto& kk, const auto& vv, const auto& valid, int nr) {
    constexpr int RA = sizeof(valid) / sizeof(valid[0]);
    float sc[RA][GQA];
#pragma unroll
    for (int r = 0; r < RA; ++r)
#pragma unroll
      for (int g = 0; g < GQA; ++g) {
        sc[r][g] = -INFINITY;
        if (r < nr) {
          const float x = sum_lanes8(dot8(kk[r], q[g], 0.f));
          sc[r][g] = valid[r] ? x * SM_SCALE : -INFINITY;
        }
      }
#pragma unroll
    for (int g = 0; g < GQA; ++g) {
      float mn = m_run[g];
#pragma unroll
      for (int r = 0; r < RA; ++r) mn = fmaxf(mn, sc[r][g]);
      const float keep = mn == -INFINITY ? 1.f : __expf(m_run[g] - mn);
      l_run[g] *= keep;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] *= keep;
#pragma unroll
      for (int r = 0; r < RA; ++r) {
        if (r >= nr) continue;
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
  // cached rows in groups of R rounds, the loads of the next group in flight while one is
  // consumed. The buffers rotate by unrolling (a register copy of a buffer whose loads are in
  // flight would wait for them), and the loads ahead are issued unconditionally (rows past the
  // item read nothing: out-of-range offsets), so the compiler's wait before each consume counts
  // exactly the loads issued after it instead of falling back to waiting for all of them.
  const int ngroups = rows.template ngroups<R>();
  // A full group (every row valid), the same arithmetic in the same order as
  // consume(), as straight-line code: without the per-round checks and masks
  // the compiler can interleave the 16 independent dot / softmax chains
  // (with the checks the loop body was split into ~35 small blocks per group).
  // MASKED: a partial group, every round computed with the invalid rows masked
  // (score -inf, weight 0; their K/V read as zero) instead of skipping rounds
  // with branches: the same results.
  auto consume_full = [&](const AttnGroupT<R>& gr, auto masked) {
    constexpr bool MASKED = decltype(masked)::value;
    float sc[R][GQA];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int g = 0; g < GQA; ++g) {
        const float x = sum_lanes8(dot8(gr.k[r], q[g], 0.f)) * SM_SCALE;
        sc[r][g] = !MASKED || gr.valid[r] ? x : -INFINITY;
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
        const float pr = !MASKED || gr.valid[r] ? __expf(sc[r][g] - mn) : 0.f;
        l_run[g] += pr;
        const uint32_t w4[4] = {gr.v[r].x, gr.v[r].y, gr.v[r].z, gr.v[r].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[g][2 * e] = fmaf(pr, bf_lo(w4[e]), acc[g][2 * e]);
          acc[g][2 * e + 1] = fmaf(pr, bf_hi(w4[e]), acc[g][2 * e + 1]);
        }
      }
      m_run[g] = mn;
    }
  };
  auto step = [&](int gi, AttnGroupT<R>& cur, AttnGroupT<R>& ahead) {
    rows.load(gi + 1, ahead);   // past the last group: all rows invalid, nothing read
    if (gi < ngroups) {
      const int left = rows.jc - rows.j0 - gi * 32 * R;   // rows of this group and beyond
      if (left >= 32 * R) consume_full(cur, BoolC<false>());
      else consume_full(cur, BoolC<true>());
    }
  };
  AttnGroupT<R>& A = first;
  AttnGroupT<R> B;
  for (int gi = 0; gi < ngroups; gi += 2) {
    step(gi, A, B);
    step(gi + 1, B, A);
  }
  if (fresh) {   // the new row: row-lane 0 of one round
    const bool valid[1] = {rl == 0};
    const u32x4 kk[1] = {valid[0] ? *reinterpret_cast<const u32x4*>(q_lds + GQA * HD + ch * 8) : u32x4{0u, 0u, 0u, 0u}};
    const u32x4 vv[1] = {valid[0] ? *reinterpret_cast<const u32x4*>(q_lds + GQA * HD + HD + ch * 8)
                                  : u32x4{0u, 0u, 0u, 0u}};
    consume(kk, vv, valid, 1);
  }
  // The loads issued ahead past the last group read nothing (out of range);
  // drain them now, while nothing else is in flight, so that no later code
  // reusing their registers waits for the stores and copies issued after them.
  wait_mem();
  // merge the 32 row-lanes of the item (lane bits 3-5 within a wave, then the
  // 4 waves through LDS): max, rescale, sum. The lanes of one row agree.
  {
    float mv[GQA];
#pragma unroll
    for (int g = 0; g < GQA; ++g) mv[g] = m_run[g];
    reduce_stride8<GQA, true>(mv);   // lane: head 2*b5 + b4
    if ((lane & 15) == 0) sh.mx[wave][lane >> 4] = mv[0];
  }
  lds_sync();
  {
    float lv[GQA], av[GQA * 8];
#pragma unroll
    for (int g = 0; g < GQA; ++g) {
      const float M = fmaxf(fmaxf(sh.mx[0][g], sh.mx[1][g]), fmaxf(sh.mx[2][g], sh.mx[3][g]));
      const float f = m_run[g] == -INFINITY ? 0.f : __expf(m_run[g] - M);
      lv[g] = l_run[g] * f;
#pragma unroll
      for (int e = 0; e < 8; ++e) av[g * 8 + e] = acc[g][e] * f;
    }
    reduce_stride8<GQA, false>(lv);       // lane: head 2*b5 + b4
    if ((lane & 15) == 0) sh.sm[wave][lane >> 4] = lv[0];
    reduce_stride8<GQA * 8, false>(av);   // lane: values 4*(lane >> 3) .. +3 of head-major [4][8]
    *reinterpret_cast<float4*>(&sh.pv[wave][ch][(lane >> 3) * 4]) = make_float4(av[0], av[1], av[2], av[3]);
  }
  lds_sync();
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
  lds_sync();   // LDS reuse by a following item
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// D = A B^T + C over one 16x16x32 bf16 tile (v_mfma_f32_16x16x32_bf16): lane l
// holds A row l%16 and B row l%16, columns (l/16)*8 .. +7 of the 32; D[i] of
// lane l is element (row 4*(l/16) + i, column l%16).
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                 0, 0, 0);
}

// K/V rows of one ATT_GROUP-row group of the MFMA attention item: wave w takes
// rows 32w .. 32w+31 of the group.
//   k[t][s]: K as MFMA A operands, 16-row tile t: lane l holds row 32w + 16t + l%16,
//            dims 32s + (l/16)*8 .. +7
//   v[r]:    V for the VALU PV product: lane l holds row 32w + 8r + l/8, dims (l%8)*8 .. +7
// Rows >= jc read zero through out-of-range offsets.
struct AttnGroupMx {
  u32x4 k[2][2];
  u32x4 v[4];
};
static_assert(ATT_GROUP == 32 * NWAVE, "a group is 32 rows per wave");
__device__ __forceinline__ void load_mx(const AttnRows& rows, int gi, AttnGroupMx& g) {
  const int lane = lane_id(), base = rows.j0 + gi * ATT_GROUP + 32 * wave_id();
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int j = base + 16 * t + (lane & 15);
#pragma unroll
    for (int s = 0; s < 2; ++s)
      g.k[t][s] = ld_stream(rows.rk, j < rows.jc ? (uint32_t)(j * HD + 32 * s + (lane >> 4) * 8) * 2u : OOB);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int j = base + 8 * r + (lane >> 3);
    g.v[r] = ld_stream(rows.rv, j < rows.jc ? (uint32_t)(j * HD + (lane & 7) * 8) * 2u : OOB);
  }
}

// The attention work item of attn_item with the scores on the matrix cores:
// same inputs, outputs and ring protocol (groups issued with load_mx).
// Per group and wave, S = K q^T is two 16x16x32 MFMA tiles per 16 rows (rows on
// M, the 4 q heads on N, q pre-scaled by 1/8, an exact power of two), so lane
// (q4 = l/16, n = l%16) holds the scores of head n (n < 4; the other columns
// are padding) for rows 16t + 4*q4 + i. The softmax runs there once per
// (row, head), against a running maximum shared by the wave; p = exp(s - m)
// stays fp32 and reaches the VALU PV product (lane: row l/8 of each 8-row
// round, dims (l%8)*8 ..) through the wave's slice of sh.pv, which the final
// merge reuses afterwards. The last arrival's merge is that of attn_item.
//
// att (optional): the item is the head's only split, and it writes the final
// output o / l (the value the merge of its one partial would give, bit for
// bit) as bf16 to row tok, columns col0 .. of a [tokens][2048] matrix in A-tile
// order instead of the partial.
template <int DEPTH = 1>
__device__ __forceinline__ void attn_item_mx(const AttnRows& rows, AttnGroupMx (&ring)[DEPTH + 1],
                                             const uint16_t* q_lds, bool fresh, float* part, AttnShared& sh,
                                             uint16_t* att = nullptr, int tok = 0, int col0 = 0) {
  const int t = tid(), wave = wave_id(), lane = lane_id(), n = lane & 15, q4 = lane >> 4;
  // B operands: q of head n (zero for the padding columns), times 1/8
  u32x4 qb[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (n < GQA) {
      const u32x4 raw = *reinterpret_cast<const u32x4*>(q_lds + n * HD + 32 * s + q4 * 8);
      const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
      uint32_t o4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) o4[e] = f2bf(bf_lo(w4[e]) * SM_SCALE) | (f2bf(bf_hi(w4[e]) * SM_SCALE) << 16);
      v = u32x4{o4[0], o4[1], o4[2], o4[3]};
    }
    qb[s] = v;
  }
  float m_run = -INFINITY, l_part = 0.f;   // head n: the wave's running max, this lane's share of the sum
  float acc[GQA][8];
#pragma unroll
  for (int g = 0; g < GQA; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  float* pw = &sh.pv[wave][0][0];   // p of the wave's 32 rows: [row][head]
  const int ngroups = rows.template ngroups<ATT_R>();
  auto consume = [&](int gi, const AttnGroupMx& gr, auto masked) {
    constexpr bool MASKED = decltype(masked)::value;
    f32x4 sc[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      sc[tt] = mfma16(gr.k[tt][0], qb[0], f32x4{0.f, 0.f, 0.f, 0.f});
      sc[tt] = mfma16(gr.k[tt][1], qb[1], sc[tt]);
    }
    if (MASKED) {
      const int rb = rows.j0 + gi * ATT_GROUP + 32 * wave + 4 * q4;
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (rb + 16 * tt + i >= rows.jc) sc[tt][i] = -INFINITY;
    }
    float gm = fmaxf(fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3])),
                     fmaxf(fmaxf(sc[1][0], sc[1][1]), fmaxf(sc[1][2], sc[1][3])));
    gm = max_xor32(max_xor16(gm));   // head n's maximum over the wave's 32 rows
    const float mn = fmaxf(m_run, gm);
    const float keep = mn == -INFINITY ? 1.f : __expf(m_run - mn);
    float p[2][4], ps = 0.f;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[tt][i] = MASKED && sc[tt][i] == -INFINITY ? 0.f : __expf(sc[tt][i] - mn);
        ps += p[tt][i];
      }
    l_part = fmaf(l_part, keep, ps);
    m_run = mn;
    if (n < GQA) {
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) pw[(16 * tt + 4 * q4 + i) * GQA + n] = p[tt][i];
    }
    float kg[GQA];
#pragma unroll
    for (int g = 0; g < GQA; ++g) kg[g] = lane_val(keep, g);
    if (kg[0] != 1.f || kg[1] != 1.f || kg[2] != 1.f || kg[3] != 1.f) {
#pragma unroll
      for (int g = 0; g < GQA; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] *= kg[g];
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float4 p4 = *reinterpret_cast<const float4*>(pw + (8 * r + (lane >> 3)) * GQA);
      const float pg[GQA] = {p4.x, p4.y, p4.z, p4.w};
      const uint32_t w4[4] = {gr.v[r].x, gr.v[r].y, gr.v[r].z, gr.v[r].w};
#pragma unroll
      for (int g = 0; g < GQA; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[g][2 * e] = fmaf(pg[g], bf_lo(w4[e]), acc[g][2 * e]);
          acc[g][2 * e + 1] = fmaf(pg[g], bf_hi(w4[e]), acc[g][2 * e + 1]);
        }
    }
  };
  auto step = [&](int gi, AttnGroupMx& cur, AttnGroupMx& ahead) {
    load_mx(rows, gi + DEPTH, ahead);   // past the last group: all rows out of range, nothing read
    if (gi < ngroups) {
      if (rows.jc - rows.j0 - gi * ATT_GROUP >= ATT_GROUP) consume(gi, cur, BoolC<false>());
      else consume(gi, cur, BoolC<true>());
    }
  };
  constexpr int NB = DEPTH + 1;
  for (int gi = 0; gi < ngroups; gi += NB) {
#pragma unroll
    for (int s = 0; s < NB; ++s) step(gi + s, ring[s], ring[(s + DEPTH) % NB]);
  }
  wait_mem();   // drain the out-of-range loads issued past the last group
  // the wave's maximum and sum of head g, in every lane
  const float l_wave = add_xor32(add_xor16(l_part));
  float mg[GQA], lg[GQA];
#pragma unroll
  for (int g = 0; g < GQA; ++g) {
    mg[g] = lane_val(m_run, g);
    lg[g] = lane_val(l_wave, g);
  }
  const int ch = t & 7;
  if (fresh && wave == 0) {   // the new row (from LDS), counted once: wave 0, row-lane 0
    const u32x4 kf = *reinterpret_cast<const u32x4*>(q_lds + GQA * HD + ch * 8);
    const u32x4 vf = *reinterpret_cast<const u32x4*>(q_lds + GQA * HD + HD + ch * 8);
    const uint32_t w4[4] = {vf.x, vf.y, vf.z, vf.w};
    const bool mine = (lane >> 3) == 0;
#pragma unroll
    for (int g = 0; g < GQA; ++g) {
      const u32x4 qv = *reinterpret_cast<const u32x4*>(q_lds + g * HD + ch * 8);
      const float x = sum_lanes8(dot8(kf, qv, 0.f)) * SM_SCALE;
      const float mn = fmaxf(mg[g], x);
      const float keep = mg[g] == -INFINITY ? 1.f : __expf(mg[g] - mn);
      const float pr = __expf(x - mn);
      lg[g] = fmaf(lg[g], keep, pr);
      mg[g] = mn;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[g][2 * e] = fmaf(mine ? pr : 0.f, bf_lo(w4[e]), acc[g][2 * e] * keep);
        acc[g][2 * e + 1] = fmaf(mine ? pr : 0.f, bf_hi(w4[e]), acc[g][2 * e + 1] * keep);
      }
    }
  }
  // merge the 8 row-lanes of each wave (lane bits 3-5), then the 4 waves through
  // LDS (each wave rewrites only its own slice of sh.pv): the wave's max is
  // uniform, its sum enters once (row-lane 0)
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < GQA; ++g) sh.mx[wave][g] = mg[g];
  }
  lds_sync();
  {
    float lv[GQA], av[GQA * 8];
#pragma unroll
    for (int g = 0; g < GQA; ++g) {
      const float M = fmaxf(fmaxf(sh.mx[0][g], sh.mx[1][g]), fmaxf(sh.mx[2][g], sh.mx[3][g]));
      const float f = mg[g] == -INFINITY ? 0.f : __expf(mg[g] - M);
      lv[g] = (lane >> 3) == 0 ? lg[g] * f : 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) av[g * 8 + e] = acc[g][e] * f;
    }
    reduce_stride8<GQA, false>(lv);       // lane: head 2*b5 + b4
    if ((lane & 15) == 0) sh.sm[wave][lane >> 4] = lv[0];
    reduce_stride8<GQA * 8, false>(av);   // lane: values 4*(lane >> 3) .. +3 of head-major [4][8]
    *reinterpret_cast<float4*>(&sh.pv[wave][ch][(lane >> 3) * 4]) = make_float4(av[0], av[1], av[2], av[3]);
  }
  lds_sync();
  {
    const int g = t >> 6, d = t & 63;
    float o = 0.f;
#pragma unroll
    for (int wv = 0; wv < NWAVE; ++wv) o += sh.pv[wv][d >> 3][g * 8 + (d & 7)];
    if (att) {
      const uint32_t mine = f2bf(o / (sh.sm[0][g] + sh.sm[1][g] + sh.sm[2][g] + sh.sm[3][g]));
      const uint32_t next = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mine, DPP_XOR1, 0xf, 0xf, false);
      if ((d & 1) == 0)
        st_dev(reinterpret_cast<uint32_t*>(att + a_tile_off(tok, col0 + g * HD + d, 2048 / 32)), mine | (next << 16));
    } else {
      st_dev(part + 2 * GQA + g * HD + d, o);
      if (t < GQA) {
        st_dev(part + t, fmaxf(fmaxf(sh.mx[0][t], sh.mx[1][t]), fmaxf(sh.mx[2][t], sh.mx[3][t])));
        st_dev(part + GQA + t, sh.sm[0][t] + sh.sm[1][t] + sh.sm[2][t] + sh.sm[3][t]);
      }
    }
  }
  lds_sync();   // LDS reuse by a following item
}

// Merge the nsplit partials of one kv head (split s at part_head + s * PART_FLOATS)
// into the bf16 attention output of its 4 q heads:
//   att = sum_s e^(m_s-M) o_s / sum_s e^(m_s-M) l_s   (then cast to bf16)
// Thread t produces q head (t >> 6) of the group, dim t & 63, at att[(t >> 6) * 64 + (t & 63)].
// POLL: the partials are polled until none holds the fp32 sentinel; otherwise
// the caller knows they are complete and they are read once (device scope).
// MAXS: the most splits a call may pass.
constexpr int ATT_MERGE_MAX = 8;   // splits the polled merge reads at most

// TILED: att is the base of a [tokens][2048] matrix in A-tile order and the
// head's 256 outputs go to row tok, columns col0 ..; otherwise att points at
// the head's 256 contiguous outputs.
template <bool POLL = true, int MAXS = ATT_MERGE_MAX, bool TILED = false>
__device__ __forceinline__ void attn_merge_head(const Sync& sy, const float* part_head, int nsplit, uint16_t* att,
                                                int tok = 0, int col0 = 0) {
  const int t = tid(), g = t >> 6, d = t & 63;
  const rsrc_t r = make_rsrc(part_head, (size_t)nsplit * PART_FLOATS * 4);
  uint32_t m[MAXS], l[MAXS], o[MAXS];
  const unsigned long long t0 = wall_clock64();
  for (int it = 1;; ++it) {
    bool ok = true;
#pragma unroll
    for (int s = 0; s < MAXS; ++s) {   // splits >= nsplit read zero (out of range)
      const uint32_t base = (uint32_t)(s * PART_FLOATS) * 4u;
      m[s] = ld_dev4(r, base + (uint32_t)g * 4u);
      l[s] = ld_dev4(r, base + (uint32_t)(GQA + g) * 4u);
      o[s] = ld_dev4(r, base + (uint32_t)(2 * GQA + g * HD + d) * 4u);
    }
    if (!POLL) break;
#pragma unroll
    for (int s = 0; s < MAXS; ++s) ok = ok && m[s] != 0xffffffffu && l[s] != 0xffffffffu && o[s] != 0xffffffffu;
    if (__all(ok)) break;
    if (wait_expired(sy, t0, it)) break;
    __builtin_amdgcn_s_sleep(1);
  }
  float M = -INFINITY;
#pragma unroll
  for (int s = 0; s < MAXS; ++s)
    if (s < nsplit) M = fmaxf(M, __uint_as_float(m[s]));
  float O = 0.f, Lsum = 0.f;
#pragma unroll
  for (int s = 0; s < MAXS; ++s) {
    const float wgt = s < nsplit ? __expf(__uint_as_float(m[s]) - M) : 0.f;
    Lsum = fmaf(wgt, __uint_as_float(l[s]), Lsum);
    O = fmaf(wgt, __uint_as_float(o[s]), O);
  }
  const uint32_t mine = f2bf(O / Lsum);
  const uint32_t next = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mine, DPP_XOR1, 0xf, 0xf, false);
  if ((d & 1) == 0) {
    uint16_t* dst = TILED ? att + a_tile_off(tok, col0 + g * HD + d, 2048 / 32) : att + g * HD + d;
    st_dev(reinterpret_cast<uint32_t*>(dst), mine | (next << 16));
  }
}

}  // namespace mk
