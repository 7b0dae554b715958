// mk_prefill.hip — context encoding (prefill) of one sequence, layer by layer,
// on the matrix cores of MI355X (gfx950).
//
// The reference encodes a prompt with its baseline decoder layers before the
// megakernel takes over token generation (llama_with_megakernel.py:194-204;
// the layer is llama.py:1039-1139). With T prompt tokens the step is T rows
// of GEMMs against every layer's weights, so it runs layer-major: each layer's
// weights stream once per chunk of up to `cap` tokens (the decode megakernel
// would stream them once per token, and its batched prefill once per 32).
//
// Per layer (all launches on the caller's stream, in order):
//   pf_norm   x -> xn = bf16(x * rsqrt(mean(x^2) + eps))      (layer 0: x = embed[token])
//   pf_gemm   QKV: xn W_qkv^T, bf16, RoPE on (d, d+32) pairs -> q; K/V rows -> the caches
//   pf_attn   causal GQA attention of every token over cache rows [0, pos] -> att
//   pf_gemm   O:    att W_o^T  + x  -> h1                       (bf16 residual add)
//   pf_norm   h1 -> xn
//   pf_gemm   GU:   xn W_gu^T, bf16(silu(g) * u) -> act
//   pf_gemm   DOWN: act W_d^T + h1 -> x (the next layer's input)
// The rounding points are those of the decode kernels (the reference's
// attention.py / mlp.py). The last layer runs only its QKV GEMM (its K/V
// rows are the prefill's output) unless the caller asks for the hidden state.
//
// GEMMs: bf16 v_mfma_f32_16x16x32_bf16 with fp32 accumulation, a 128x128
// output tile per 256-thread workgroup, 64x64 per wave (16 MFMA tiles). The
// activations are kept in A-tile order (the producing kernel writes them so)
// and the weights are the MFMA-tiled copies, so each k-step's operands of the
// tile are 16 blocks of 1 KiB, which the four waves copy from memory straight
// into LDS (one contiguous 1 KiB copy each, four per wave) three k-steps ahead
// of their use; each wave reads its 4 A and 4 B operands of a k-step from LDS
// (a block per instruction, conflict-free) and runs 16 MFMAs. The O and down
// projections of short prompts (few row tiles) split K across workgroups into
// fp32 partials that pf_reduce_norm sums in a fixed order; so does the QKV
// projection, whose tail (pf_qkv_finish) then applies RoPE and scatters.
//
// Attention: per (kv head, block of 16 tokens) one workgroup; S^T = K Q^T on
// the matrix cores (keys on M, the 16 tokens x 4 q heads on N), an online
// softmax per (token, head) column, and O^T = V^T P^T on the matrix cores with
// p rounded to bf16 as the reference rounds it (relative to the running
// maximum). K and V tiles of 32 keys go through LDS (V transposed there).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "mk.h"
#include "mk_common.h"
#include "mk_prefill.h"

namespace {

using namespace mk;

constexpr int PF_TM = 128, PF_TN = 128;   // GEMM output tile per workgroup
constexpr int PF_TB = 16;                 // tokens per attention workgroup

enum : int { EPI_QKV = 0, EPI_RES = 1, EPI_SWIGLU = 2, EPI_PART = 3 };
constexpr int GEMM_NS = 4;   // k-steps of operands in flight per wave (a ring of register stages)

struct GemmArgs {
  const uint16_t* a;     // activations, A-tile order [M16][K]
  const uint16_t* b;     // weights [N][K]: MFMA tile order (tiled) or row-major
  int tiled;
  int M, N, K;
  int splits;            // EPI_PART: the K range is cut into `splits` parts (blockIdx.y)
  const uint16_t* res;   // EPI_RES: residual, row-major [M][N]
  uint16_t* out;         // EPI_RES: row-major [M][N]; EPI_SWIGLU: A-tile order [M16][N/2]; EPI_QKV: q [M][2048]
  float* part;           // EPI_PART: fp32 [splits][M][N]
  uint16_t* kc;          // EPI_QKV: the layer's caches, bf16 [8][s_max][64]
  uint16_t* vc;
  const uint16_t* rope;  // bf16 [rows][128]
  int s_max, p0;
};

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// One k-step of a workgroup's 128x128 tile in LDS: the 8 A blocks (16 rows x
// 32 columns each, 1 KiB, MFMA A-operand lane order) and the 8 B blocks.
struct GemmStage {
  u32x4 a[8][64];
  u32x4 b[8][64];
};
struct GemmLds {
  GemmStage st[GEMM_NS];
};
// The epilogue's side input in LDS: PF_TM rows of 128 bf16, padded to 136
// (a 272-byte row stride spreads the rows of one read over the banks).
constexpr int SIDE_LD = 136;
static_assert(PF_TM * SIDE_LD * 2 <= (int)sizeof(GemmLds), "side input over the operand stages");

template <int EPI>
__global__ void __launch_bounds__(NT) pf_gemm(GemmArgs g) {
  __shared__ GemmLds L;
  const int wave = __builtin_amdgcn_readfirstlane(wave_id()), lane = lane_id();   // (uniform: LDS copy bases)
  const int nbn = g.N / PF_TN;
  const int tm = blockIdx.x / nbn, tn = blockIdx.x % nbn;
  const int m16 = (g.M + 15) / 16;
  const rsrc_t ra = make_rsrc(g.a, (size_t)m16 * 16 * g.K * 2);
  const rsrc_t rb = make_rsrc(g.b, (size_t)g.N * g.K * 2);
  // the k-steps of this workgroup: all of K, or part blockIdx.y of `splits`
  const int kb = g.K / 32, kn = EPI == EPI_PART ? kb / g.splits : kb;
  const int k0 = EPI == EPI_PART ? (int)blockIdx.y * kn : 0, ke = k0 + kn;   // kn: a multiple of GEMM_NS
  // Staging: wave w copies A blocks 2w, 2w+1 and B blocks 2w, 2w+1 of each
  // k-step from memory straight into LDS (one 1 KiB copy each); k-steps
  // >= ke copy zeros from out-of-range offsets (no memory read).
  const int ab0 = tm * 8 + 2 * wave, bb0 = tn * 8 + 2 * wave;
  auto issue = [&](int ks, int stg) {
    const bool kin = ks < ke;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const uint32_t ao = kin ? (uint32_t)(((size_t)(ab0 + u) * kb + ks) * 1024 + lane * 16) : OOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)&L.st[stg].a[2 * wave + u][0], 16, ao, 0, 0, 0);
      uint32_t bo = OOB;
      if (kin)
        bo = g.tiled ? (uint32_t)(((size_t)(bb0 + u) * kb + ks) * 1024 + lane * 16)
                     : (uint32_t)((((size_t)(bb0 + u) * 16 + (lane & 15)) * g.K + ks * 32 + (lane >> 4) * 8) * 2);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr_t)&L.st[stg].b[2 * wave + u][0], 16, bo, 0, 0, 0);
    }
  };
  // The epilogue's side input, 128 rows of 256 bytes: the RoPE rows of the
  // tile's tokens (EPI_QKV) or the residual tile (EPI_RES). Two threads per
  // row load it with 16-byte loads before the first operand copies (so they
  // are the oldest loads in flight and land first); it goes to LDS after the
  // k-loop, so the epilogue reads LDS instead of waiting on a 2-byte global
  // load per element. Rows past the tokens read zero.
  constexpr bool SIDE = EPI == EPI_QKV || EPI == EPI_RES;
  const int srow = threadIdx.x >> 1, shalf = threadIdx.x & 1;
  u32x4 side[SIDE ? 8 : 1];
  if constexpr (SIDE) {
    const int m = tm * PF_TM + srow;
    rsrc_t rs;
    uint32_t off = OOB;
    if constexpr (EPI == EPI_RES) {
      rs = make_rsrc(g.res, (size_t)g.M * g.N * 2);
      if (m < g.M) off = (uint32_t)(((size_t)m * g.N + (size_t)tn * PF_TN) * 2) + (uint32_t)shalf * 128u;
    } else {
      rs = make_rsrc(g.rope, (size_t)g.s_max * (4 * HD));
      if (m < g.M) off = (uint32_t)((size_t)(g.p0 + m) * (4 * HD)) + (uint32_t)shalf * 128u;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) side[k] = ld16(rs, off == OOB ? OOB : off + 16u * (uint32_t)k);
  }
  // wave (wm, wn) computes rows 64*wm .. +63 and columns 64*wn .. +63 of the tile
  const int wm = wave & 1, wn = wave >> 1;
  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < GEMM_NS - 1; ++s) issue(k0 + s, s);
  for (int ks = k0; ks < ke; ks += GEMM_NS) {
#pragma unroll
    for (int s = 0; s < GEMM_NS; ++s) {
      // this wave's copies of stage s have landed (the GEMM_NS - 2 later
      // stages' 4 copies each may be in flight; the side loads, issued
      // first, have landed too), and, after the barrier, every wave's; every
      // wave has also finished reading the stage refilled next
      static_assert(GEMM_NS == 4, "the wait below counts 2 later stages of 4 copies");
      asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
      issue(ks + s + GEMM_NS - 1, (s + GEMM_NS - 1) % GEMM_NS);
      const GemmStage& S = L.st[s];
      u32x4 av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = S.a[4 * wm + i][lane];
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = S.b[4 * wn + j][lane];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16(av[i], bv[j], acc[i][j]);
    }
  }
  const int am = tm * 8 + 4 * wm, bn = tn * 8 + 4 * wn;   // the wave's first A / B tile
  // the side input into LDS, over the operand stages: every wave's operand
  // reads and copies (the trailing ones write zeros into the stages) are done
  const uint16_t* side_lds = reinterpret_cast<const uint16_t*>(&L);   // [PF_TM][SIDE_LD]
  if constexpr (SIDE) {
    __syncthreads();
    u32x4* dst = reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(&L) + srow * SIDE_LD + shalf * 64);
#pragma unroll
    for (int k = 0; k < 8; ++k) dst[k] = side[k];
    __syncthreads();
  }

  // epilogue: acc[i][j][r] is (row 16*(am+i) + 4*(lane/16) + r, column 16*(bn+j) + lane%16)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = 16 * (bn + j) + (lane & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 16 * (am + i) + 4 * (lane >> 4) + r;
        const float v = acc[i][j][r];
        if constexpr (EPI == EPI_PART) {
          if (m < g.M) g.part[((size_t)blockIdx.y * g.M + m) * g.N + n] = v;
        } else if constexpr (EPI == EPI_RES) {
          if (m < g.M) {
            const uint16_t r0 = side_lds[(m - tm * PF_TM) * SIDE_LD + (n - tn * PF_TN)];
            g.out[(size_t)m * g.N + n] = (uint16_t)f2bf(bf2f(r0) + rbf(v));
          }
        } else if constexpr (EPI == EPI_SWIGLU) {
          // rows (gate_i, up_i) interleaved: lanes 2k (gate) and 2k+1 (up)
          const float u = dpp<DPP_XOR1>(v);
          if (m < g.M && (lane & 1) == 0)
            g.out[a_tile_off(m, n >> 1, g.N / 64)] = (uint16_t)f2bf(v / (1.0f + __expf(-v)) * u);
        } else {
          // q, k, v rows in RoPE pairs (d, d+32): lanes 2k (d) and 2k+1 (d+32)
          const float x = rbf(v);
          const float y = dpp<DPP_XOR1>(x);
          if (m < g.M) {
            const int pair = n >> 1, e = n & 1, pos = g.p0 + m;
            const int hp = pair & 31;                      // d = hp + 32e
            const uint16_t* rrow = side_lds + (m - tm * PF_TM) * SIDE_LD;   // row pos of the RoPE table
            float o = x;
            if (pair < Q_PAIRS + K_PAIRS) {
              const float a = e ? y : x, b = e ? x : y;    // the pair (x[d], x[d+32])
              const int d = hp + 32 * e;
              const float c = bf2f(rrow[d]), s = bf2f(rrow[HD + d]);
              o = e ? rbf(rbf(b * c) + rbf(a * s)) : rbf(rbf(a * c) + rbf(-b * s));
            }
            const uint16_t ob = (uint16_t)f2bf(o);
            const int d = hp + 32 * e;
            if (pair < Q_PAIRS) {
              g.out[(size_t)m * H + (pair >> 5) * HD + d] = ob;
            } else if (pair < Q_PAIRS + K_PAIRS) {
              g.kc[((size_t)((pair - Q_PAIRS) >> 5) * g.s_max + pos) * HD + d] = ob;
            } else {
              g.vc[((size_t)((pair - Q_PAIRS - K_PAIRS) >> 5) * g.s_max + pos) * HD + d] = ob;
            }
          }
        }
      }
    }
  }
}

// The split-K tail of the O and down projections (N = 2048), one 64-thread
// workgroup per token row t (the rows spread over every CU): v = the sum of
// the SPLITS fp32 partials in split order, out = bf16(res + bf16(v))
// (row-major), and, if xn is given, the next RMSNorm of out into xn (A-tile
// order), as pf_norm computes it. Every partial of a group of chunks is
// loaded before the first sum, so the loads overlap instead of waiting one
// split at a time.
template <int SPLITS>
__global__ void __launch_bounds__(64) pf_reduce_norm(const float* part, const uint16_t* res, uint16_t* out,
                                                     uint16_t* xn, int T) {
  const int t = blockIdx.x, lane = lane_id();
  if (t >= T) return;
  constexpr int CH = SPLITS <= 4 ? 4 : (SPLITS <= 8 ? 2 : 1);   // 512-column chunks loaded at once
  u32x4 xs[4];
#pragma unroll
  for (int i0 = 0; i0 < 4; i0 += CH) {
    float4 pv[CH][SPLITS][2];
    u32x4 rv[CH];
#pragma unroll
    for (int ci = 0; ci < CH; ++ci) {
      const int c = (i0 + ci) * 512 + lane * 8;
#pragma unroll
      for (int sp = 0; sp < SPLITS; ++sp) {
        const float4* pp = reinterpret_cast<const float4*>(part + ((size_t)sp * T + t) * H + c);
        pv[ci][sp][0] = pp[0];
        pv[ci][sp][1] = pp[1];
      }
      rv[ci] = *reinterpret_cast<const u32x4*>(res + (size_t)t * H + c);
    }
#pragma unroll
    for (int ci = 0; ci < CH; ++ci) {
      float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int sp = 0; sp < SPLITS; ++sp) {
        const float4 p0 = pv[ci][sp][0], p1 = pv[ci][sp][1];
        v[0] += p0.x; v[1] += p0.y; v[2] += p0.z; v[3] += p0.w;
        v[4] += p1.x; v[5] += p1.y; v[6] += p1.z; v[7] += p1.w;
      }
      const uint32_t rw[4] = {rv[ci].x, rv[ci].y, rv[ci].z, rv[ci].w};
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o[e] = f2bf(bf_lo(rw[e]) + rbf(v[2 * e])) | (f2bf(bf_hi(rw[e]) + rbf(v[2 * e + 1])) << 16);
      const int i = i0 + ci;
      xs[i] = u32x4{o[0], o[1], o[2], o[3]};
      *reinterpret_cast<u32x4*>(out + (size_t)t * H + i * 512 + lane * 8) = xs[i];
    }
  }
  if (!xn) return;
  rmsnorm2048(xs, nullptr);
#pragma unroll
  for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(xn + a_tile_off(t, i * 512 + lane * 8, H / 32)) = xs[i];
}

// The split-K tail of the QKV projection of short prompts (N = 3072): thread
// (t, j) takes RoPE pairs 2j and 2j + 1 of token row t, i.e. columns 4j .. 4j + 3
// (dims d, d + 32, d + 1, d + 33 of one head, d = 2j mod 32), in one 16-byte
// load per split: each column summed over the SPLITS fp32 partials in split
// order and rounded to bf16, RoPE on the q and k pairs as the QKV GEMM's
// epilogue does it, q to the q buffer and k and v to the caches at row
// p0 + t, two bf16 per 4-byte store. Grid (T, QKV_PAIRS / 2 / NT).
template <int SPLITS>
__global__ void __launch_bounds__(NT) pf_qkv_finish(const float* part, const uint16_t* rope, uint16_t* q,
                                                    uint16_t* kc, uint16_t* vc, int T, int p0, int s_max) {
  const int t = blockIdx.x, j = blockIdx.y * NT + (int)threadIdx.x;
  if (t >= T || j >= QKV_PAIRS / 2) return;
  const int pos = p0 + t, pr = 2 * j, hp = pr & 31;
  float4 pv[SPLITS];
#pragma unroll
  for (int sp = 0; sp < SPLITS; ++sp)
    pv[sp] = *reinterpret_cast<const float4*>(part + ((size_t)sp * T + t) * QKV_ROWS + 4 * j);
  float v0 = 0.f, v1 = 0.f, v2 = 0.f, v3 = 0.f;
#pragma unroll
  for (int sp = 0; sp < SPLITS; ++sp) {
    v0 += pv[sp].x;
    v1 += pv[sp].y;
    v2 += pv[sp].z;
    v3 += pv[sp].w;
  }
  // pair 2j: (x[d], x[d + 32]) = (a0, b0); pair 2j + 1: (x[d + 1], x[d + 33]) = (a1, b1)
  const float a0 = rbf(v0), b0 = rbf(v1), a1 = rbf(v2), b1 = rbf(v3);
  float o00 = a0, o01 = b0, o10 = a1, o11 = b1;
  if (pr < Q_PAIRS + K_PAIRS) {
    const uint16_t* rrow = rope + (size_t)pos * (2 * HD);
    const uint32_t c0 = *reinterpret_cast<const uint32_t*>(rrow + hp);            // cos[d], cos[d + 1]
    const uint32_t s0 = *reinterpret_cast<const uint32_t*>(rrow + HD + hp);       // sin[d], sin[d + 1]
    const uint32_t c1 = *reinterpret_cast<const uint32_t*>(rrow + hp + 32);       // cos[d + 32], ...
    const uint32_t s1 = *reinterpret_cast<const uint32_t*>(rrow + HD + hp + 32);  // sin[d + 32], ...
    o00 = rbf(rbf(a0 * bf_lo(c0)) + rbf(-b0 * bf_lo(s0)));
    o01 = rbf(rbf(b0 * bf_lo(c1)) + rbf(a0 * bf_lo(s1)));
    o10 = rbf(rbf(a1 * bf_hi(c0)) + rbf(-b1 * bf_hi(s0)));
    o11 = rbf(rbf(b1 * bf_hi(c1)) + rbf(a1 * bf_hi(s1)));
  }
  uint16_t* dst;
  if (pr < Q_PAIRS) dst = q + (size_t)t * H + (pr >> 5) * HD;
  else if (pr < Q_PAIRS + K_PAIRS) dst = kc + ((size_t)((pr - Q_PAIRS) >> 5) * s_max + pos) * HD;
  else dst = vc + ((size_t)((pr - Q_PAIRS - K_PAIRS) >> 5) * s_max + pos) * HD;
  *reinterpret_cast<uint32_t*>(dst + hp) = pack_bf2(o00, o10);
  *reinterpret_cast<uint32_t*>(dst + hp + 32) = pack_bf2(o01, o11);
}

// xn (A-tile order [T16][2048]) = bf16(x * rsqrt(mean(x^2) + eps)) per token
// row, one wave per token; with `tokens`, x is the embedding row of the token
// and is also copied to x_out (row-major) as the first residual.
__global__ void __launch_bounds__(NT) pf_norm(const uint16_t* x, const int32_t* tokens, const uint16_t* embed,
                                              uint16_t* x_out, uint16_t* xn, int T) {
  const int t = blockIdx.x * NWAVE + wave_id(), lane = lane_id();
  if (t >= T) return;
  const uint16_t* src = x + (size_t)t * H;
  if (tokens) {
    int tok = tokens[t];
    tok = tok < 0 ? 0 : (tok >= VOCAB ? VOCAB - 1 : tok);
    src = embed + (size_t)tok * H;
  }
  u32x4 xs[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) xs[i] = *reinterpret_cast<const u32x4*>(src + i * 512 + lane * 8);
  if (tokens) {
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(x_out + (size_t)t * H + i * 512 + lane * 8) = xs[i];
  }
  rmsnorm2048(xs, nullptr);
#pragma unroll
  for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(xn + a_tile_off(t, i * 512 + lane * 8, H / 32)) = xs[i];
}

struct AttnArgs {
  const uint16_t* q;     // [T][2048] row-major, after RoPE
  const uint16_t* kc;    // the layer's caches bf16 [8][s_max][64]
  const uint16_t* vc;
  uint16_t* att;         // A-tile order [T16][2048]
  int T, p0, s_max;
};

constexpr int KS_STRIDE = HD + 8;   // K tile row in LDS (bf16): 144 bytes, rows on distinct banks
constexpr int VT_STRIDE = 32 + 4;   // transposed V tile row (one dim, 32 keys): 72 bytes

struct AttnLds {
  uint16_t k[2][32][KS_STRIDE];
  uint16_t vt[2][HD][VT_STRIDE];
};

// Token t of the sequence (position p0 + t) attends to cache rows [0, p0 + t],
// its own row included (written by the QKV GEMM before this launch).
__global__ void __launch_bounds__(NT) pf_attn(AttnArgs a) {
  __shared__ AttnLds L;
  const int tid = threadIdx.x, wave = wave_id(), lane = lane_id();
  const int nblk = (a.T + PF_TB - 1) / PF_TB;
  const int tb = nblk - 1 - (int)blockIdx.x;   // the longest blocks first
  const int g = blockIdx.y;                    // kv head
  const int t0 = tb * PF_TB;
  const int n_keys = a.p0 + min(t0 + PF_TB, a.T);
  // this lane's column: token t0 + 4*wave + (lane%16)/4, q head 4g + lane%4
  const int col = lane & 15, q4 = lane >> 4;
  const int tq = t0 + 4 * wave + (col >> 2);
  const int hq = GQA * g + (col & 3);
  const int lim = a.p0 + min(tq, a.T - 1);     // last key of the column (padding tokens: any finite row)
  const rsrc_t rq = make_rsrc(a.q, (size_t)a.T * H * 2);
  u32x4 qv[2];
#pragma unroll
  for (int s = 0; s < 2; ++s)
    qv[s] = ld16(rq, tq < a.T ? (uint32_t)(((size_t)tq * H + hq * HD + 32 * s + q4 * 8) * 2) : OOB);
  const rsrc_t rk = make_rsrc(a.kc + (size_t)g * a.s_max * HD, (size_t)a.s_max * HD * 2);
  const rsrc_t rv = make_rsrc(a.vc + (size_t)g * a.s_max * HD, (size_t)a.s_max * HD * 2);
  // staging of a 32-key block: thread t loads key row t/8, dims (t%8)*8 .. +7 of K and of V
  const int sr = tid >> 3, sc = tid & 7;
  auto load_blk = [&](int kb, u32x4& kk, u32x4& vv) {
    const int key = kb * 32 + sr;
    const uint32_t off = key < n_keys ? (uint32_t)((key * HD + sc * 8) * 2) : OOB;
    kk = ld16(rk, off);
    vv = ld16(rv, off);
  };
  auto store_blk = [&](int buf, const u32x4& kk, const u32x4& vv) {
    *reinterpret_cast<u32x4*>(&L.k[buf][sr][sc * 8]) = kk;
    const uint32_t w[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      L.vt[buf][sc * 8 + 2 * e][sr] = (uint16_t)(w[e] & 0xffffu);
      L.vt[buf][sc * 8 + 2 * e + 1][sr] = (uint16_t)(w[e] >> 16);
    }
  };
  const int nb = (n_keys + 31) / 32;
  {
    u32x4 kk, vv;
    load_blk(0, kk, vv);
    store_blk(0, kk, vv);
  }
  __syncthreads();
  f32x4 acc[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) acc[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;
  for (int kb = 0; kb < nb; ++kb) {
    const int buf = kb & 1;
    u32x4 kk, vv;
    const bool more = kb + 1 < nb;
    if (more) load_blk(kb + 1, kk, vv);
    // S^T: keys 16*ks + 4*q4 + i of the block, this lane's column
    float sc4[2][4];
    float mb = -INFINITY;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int sd = 0; sd < 2; ++sd) {
        const u32x4 ko = *reinterpret_cast<const u32x4*>(&L.k[buf][16 * ks + col][32 * sd + q4 * 8]);
        s = mfma16(ko, qv[sd], s);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = kb * 32 + 16 * ks + 4 * q4 + i;
        const float v = key <= lim ? s[i] * SM_SCALE : -INFINITY;
        sc4[ks][i] = v;
        mb = fmaxf(mb, v);
      }
    }
    mb = max_xor32(max_xor16(mb));          // the column's maximum over the 32 keys
    const float m_new = fmaxf(m_run, mb);   // finite: key 0 is in every column's range
    const float alpha = __expf(m_run - m_new);
    m_run = m_new;
    float ps = 0.f;
    float p[2][4];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[ks][i] = __expf(sc4[ks][i] - m_new);
        ps += p[ks][i];
      }
    l_run = l_run * alpha + ps;
    // P^T as the B operand: k-slots 8*q4 .. +7 of lane (q4, col) are the keys
    // 4*q4 + i and 16 + 4*q4 + i it holds (the V^T operand uses the same key order)
    const u32x4 pb = {cvt_bf2(p[0][0], p[0][1]), cvt_bf2(p[0][2], p[0][3]), cvt_bf2(p[1][0], p[1][1]),
                      cvt_bf2(p[1][2], p[1][3])};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint16_t* vrow = &L.vt[buf][16 * d + col][0];
      const uint2 lo = *reinterpret_cast<const uint2*>(vrow + 4 * q4);
      const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 16 + 4 * q4);
      const u32x4 vo = {lo.x, lo.y, hi.x, hi.y};
      f32x4 c = acc[d];
#pragma unroll
      for (int i = 0; i < 4; ++i) c[i] *= alpha;
      acc[d] = mfma16(vo, pb, c);
    }
    if (more) store_blk(buf ^ 1, kk, vv);
    __syncthreads();
  }
  // the column's sum over its four lanes; o = acc / l, dims 16d + 4*q4 + i
  const float l_tot = add_xor32(add_xor16(l_run));
  const float inv = 1.0f / l_tot;
  if (tq < a.T) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int dim = 16 * d + 4 * q4;
      uint2 w;
      w.x = pack_bf2(acc[d][0] * inv, acc[d][1] * inv);
      w.y = pack_bf2(acc[d][2] * inv, acc[d][3] * inv);
      *reinterpret_cast<uint2*>(a.att + a_tile_off(tq, hq * HD + dim, H / 32)) = w;
    }
  }
}

size_t ws_per_token() { return (size_t)H * 2 * 5 + (size_t)INTER * 2; }
// fp32 partials of a split-K projection with N = 2048: splits * M <= 16 * PF_TM rows
constexpr int PART_ROWS = 16 * PF_TM;
constexpr size_t PART_BYTES = (size_t)PART_ROWS * H * 4;

// K splits of an N = 2048 projection over mt row tiles: enough workgroups
// (16 column tiles each) to occupy the device, 1 when mt alone does it.
int res_splits(int mt, int kb) {
  int s = 1;
  while (mt * s * 2 <= 16 && (kb / (s * 2)) % GEMM_NS == 0) s *= 2;
  return s;
}

// K splits of the QKV projection (N = 3072, 24 column tiles) over mt row
// tiles: up to one round of the 256-CU grid, the partials within PART_BYTES.
int qkv_splits(int mt) {
  int s = 1;
  while (mt * (QKV_ROWS / PF_TN) * s * 2 <= 256 && ((H / 32) / (s * 2)) % GEMM_NS == 0 &&
         (size_t)s * 2 * mt * PF_TM * QKV_ROWS * 4 <= PART_BYTES)
    s *= 2;
  return s;
}

}  // namespace

namespace mk {

size_t prefill_ws_bytes(int tokens) {
  const size_t t16 = (size_t)(tokens + 15) / 16 * 16;
  return t16 * ws_per_token() + PART_BYTES + 256;
}

int prefill_chunk_cap(size_t bytes) {
  if (bytes < prefill_ws_bytes(16)) return 0;
  const size_t t = (bytes - 256 - PART_BYTES) / ws_per_token() / 16 * 16;
  return t > (size_t)PREFILL_MAX_CHUNK ? PREFILL_MAX_CHUNK : (int)t;
}

hipError_t prefill_launch(const mk_weights* w, const mk_prefill_args* a, int cap) {
  hipStream_t st = static_cast<hipStream_t>(a->stream);
  const bool tiled = w->t_qkv && w->t_o && w->t_gu && w->t_down;
  const uint16_t* Wqkv = static_cast<const uint16_t*>(tiled ? w->t_qkv : w->w_qkv);
  const uint16_t* Wo = static_cast<const uint16_t*>(tiled ? w->t_o : w->w_o);
  const uint16_t* Wgu = static_cast<const uint16_t*>(tiled ? w->t_gu : w->w_gu);
  const uint16_t* Wd = static_cast<const uint16_t*>(tiled ? w->t_down : w->w_down);
  const size_t c16 = (size_t)(cap + 15) / 16 * 16;
  uint8_t* base = static_cast<uint8_t*>(a->workspace);
  uint16_t* x = reinterpret_cast<uint16_t*>(base);
  uint16_t* h1 = x + c16 * H;
  uint16_t* q = h1 + c16 * H;
  uint16_t* xn = q + c16 * H;
  uint16_t* att = xn + c16 * H;
  uint16_t* act = att + c16 * H;
  float* part = reinterpret_cast<float*>(act + c16 * INTER);
  const int L = a->n_layers, l0 = a->first_layer;
  // An N = 2048 projection (O: K = 2048, down: K = 8192) of T tokens with the
  // residual add, followed by the RMSNorm of its output into xn if `norm`:
  // as one GEMM with the add in its epilogue plus pf_norm when its 16 x mt
  // workgroups occupy the device, else split over K into fp32 partials that
  // pf_reduce_norm sums (in split order), adds and normalises.
  auto res_gemm = [&](GemmArgs g, const uint16_t* res, uint16_t* out, bool norm, int T, int mt) {
    const int sp = res_splits(mt, g.K / 32);
    const dim3 tg((unsigned)((T + NWAVE - 1) / NWAVE));
    if (sp == 1) {
      g.res = res;
      g.out = out;
      hipLaunchKernelGGL(pf_gemm<EPI_RES>, dim3(mt * (H / PF_TN)), dim3(NT), 0, st, g);
      if (norm)
        hipLaunchKernelGGL(pf_norm, tg, dim3(NT), 0, st, (const uint16_t*)out, (const int32_t*)nullptr,
                           (const uint16_t*)nullptr, (uint16_t*)nullptr, xn, T);
    } else {
      g.splits = sp;
      g.part = part;
      hipLaunchKernelGGL(pf_gemm<EPI_PART>, dim3(mt * (H / PF_TN), sp), dim3(NT), 0, st, g);
      uint16_t* xn_out = norm ? xn : nullptr;
      switch (sp) {   // res_splits gives 2, 4, 8 or 16
        case 2: hipLaunchKernelGGL(pf_reduce_norm<2>, dim3(T), dim3(64), 0, st, (const float*)part, res, out, xn_out, T); break;
        case 4: hipLaunchKernelGGL(pf_reduce_norm<4>, dim3(T), dim3(64), 0, st, (const float*)part, res, out, xn_out, T); break;
        case 8: hipLaunchKernelGGL(pf_reduce_norm<8>, dim3(T), dim3(64), 0, st, (const float*)part, res, out, xn_out, T); break;
        default: hipLaunchKernelGGL(pf_reduce_norm<16>, dim3(T), dim3(64), 0, st, (const float*)part, res, out, xn_out, T); break;
      }
    }
  };
  // Every chunk starts again from the embeddings of its own tokens; the rows
  // of earlier chunks are in the caches by then. A chunk's last layer needs
  // only its QKV GEMM unless the hidden state is asked for.
  for (int c0 = 0; c0 < a->n_tokens; c0 += cap) {
    const int T = min(cap, a->n_tokens - c0), p0 = a->start_pos + c0;
    const int mt = (T + PF_TM - 1) / PF_TM;
    hipLaunchKernelGGL(pf_norm, dim3((T + NWAVE - 1) / NWAVE), dim3(NT), 0, st, (const uint16_t*)nullptr,
                       a->tokens + c0, static_cast<const uint16_t*>(w->embed), x, xn, T);
    for (int li = 0; li < L; ++li) {
      const int l = l0 + li;
      const bool tail = li == L - 1 && !a->hidden_out;
      GemmArgs g;
      memset(&g, 0, sizeof(g));
      g.tiled = tiled;
      g.M = T;
      g.splits = 1;
      g.rope = static_cast<const uint16_t*>(w->rope);
      g.s_max = a->s_max;
      g.p0 = p0;
      uint16_t* kc = static_cast<uint16_t*>(a->k_cache[li]);
      uint16_t* vc = static_cast<uint16_t*>(a->v_cache[li]);
      // QKV + RoPE; K/V rows into the caches
      g.a = xn;
      g.b = Wqkv + (size_t)l * QKV_ROWS * H;
      g.N = QKV_ROWS;
      g.K = H;
      g.out = q;
      g.kc = kc;
      g.vc = vc;
      const int qs = qkv_splits(mt);
      if (qs == 1) {
        hipLaunchKernelGGL(pf_gemm<EPI_QKV>, dim3(mt * (QKV_ROWS / PF_TN)), dim3(NT), 0, st, g);
      } else {   // short prompts: split over K, RoPE and the scatter in the tail
        g.splits = qs;
        g.part = part;
        hipLaunchKernelGGL(pf_gemm<EPI_PART>, dim3(mt * (QKV_ROWS / PF_TN), qs), dim3(NT), 0, st, g);
        const uint16_t* rope = static_cast<const uint16_t*>(w->rope);
        switch (qs) {   // qkv_splits gives 2, 4 or 8
          case 2: hipLaunchKernelGGL(pf_qkv_finish<2>, dim3(T, QKV_PAIRS / 2 / NT), dim3(NT), 0, st, (const float*)part, rope, q, kc, vc, T, p0, a->s_max); break;
          case 4: hipLaunchKernelGGL(pf_qkv_finish<4>, dim3(T, QKV_PAIRS / 2 / NT), dim3(NT), 0, st, (const float*)part, rope, q, kc, vc, T, p0, a->s_max); break;
          default: hipLaunchKernelGGL(pf_qkv_finish<8>, dim3(T, QKV_PAIRS / 2 / NT), dim3(NT), 0, st, (const float*)part, rope, q, kc, vc, T, p0, a->s_max); break;
        }
        g.splits = 1;
      }
      if (tail) break;   // the last layer's K/V rows are all the caller needs
      AttnArgs aa;
      aa.q = q;
      aa.kc = kc;
      aa.vc = vc;
      aa.att = att;
      aa.T = T;
      aa.p0 = p0;
      aa.s_max = a->s_max;
      hipLaunchKernelGGL(pf_attn, dim3((T + PF_TB - 1) / PF_TB, NKV), dim3(NT), 0, st, aa);
      // O projection + residual -> h1, its RMSNorm -> xn
      g.a = att;
      g.b = Wo + (size_t)l * H * H;
      g.N = H;
      g.K = H;
      g.kc = g.vc = nullptr;
      res_gemm(g, x, h1, true, T, mt);
      // gate/up + SwiGLU -> act
      g.a = xn;
      g.b = Wgu + (size_t)l * 2 * INTER * H;
      g.N = 2 * INTER;
      g.K = H;
      g.out = act;
      hipLaunchKernelGGL(pf_gemm<EPI_SWIGLU>, dim3(mt * (2 * INTER / PF_TN)), dim3(NT), 0, st, g);
      // down projection + residual -> x (the next layer's input), its RMSNorm -> xn
      g.a = act;
      g.b = Wd + (size_t)l * H * INTER;
      g.N = H;
      g.K = INTER;
      res_gemm(g, h1, x, li + 1 < L, T, mt);
    }
    if (a->hidden_out) {
      const hipError_t e = hipMemcpyAsync(static_cast<uint16_t*>(a->hidden_out) + (size_t)c0 * H, x,
                                          (size_t)T * H * 2, hipMemcpyDeviceToDevice, st);
      if (e != hipSuccess) return e;
    }
  }
  return hipGetLastError();
}

}  // namespace mk
