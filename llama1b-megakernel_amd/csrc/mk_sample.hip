// mk_sample.hip — on-device sampling of the next token from the decode
// step's fp32 logits (libmk.so, MI355X / gfx950).
//
// The reference exposes sampling through NxDI's on-device sampler:
// --top-k / --top-p / --temperature / --global-topk / --on-device-sampling
// (main.py:57-61, 85, 129-130) with per-sequence parameters built by
// prepare_sampling_params(batch_size, top_k, top_p, temperature)
// (main.py:195-206). HF generation semantics are followed:
//   * greedy (top_k == 1, or temperature <= 0): the argmax, lowest index on ties;
//   * otherwise: x = logits / temperature; keep every token whose x is >= the
//     top_k-th largest x (ties at the threshold kept, as TopKLogitsWarper);
//     top_k <= 0 or > MK_SAMPLE_MAX_TOPK means the global cap
//     MK_SAMPLE_MAX_TOPK (NxDI's global top-k); then nucleus filtering over
//     the kept tokens' softmax: in descending order, a token is kept while
//     the probability mass before it is < top_p (TopPLogitsWarper: the top
//     token always stays); then a draw from the renormalised distribution.
// The draw is an inverse CDF over the kept tokens in descending order of x
// (ties by ascending index) with u = Philox4x32-10(key = seed, counter =
// (counter[row], row, 0, 0)), first output word >> 8 times 2^-24. Passing a
// sequence's position as its counter gives every step of every sequence its
// own reproducible u with no RNG state on the device.
//
// One 1024-thread workgroup per row:
//   1. radix select (4 passes of 8-bit count histograms over order-preserving
//      integer keys of the logits: dividing by temperature > 0 keeps the
//      order) finds the top_k-th largest key exactly;
//   2. the tokens at or above it are gathered into LDS and bitonic-sorted
//      (descending key, ascending index), at most MK_SAMPLE_CAND of them;
//   3. softmax numerators in that order, an inclusive prefix sum (fixed tree:
//      bitwise repeatable), the nucleus cut and the draw.
// The row (128256 fp32, 501 KB) is read from memory once per radix pass; it
// stays in the XCD's L2 after the first.
#include <hip/hip_runtime.h>

#include <stdint.h>
#include <string.h>

#include "mk.h"

namespace {

constexpr int ST = 1024;                 // threads per workgroup
constexpr int CAND = MK_SAMPLE_CAND;     // candidate slots (top-k set incl. ties)
constexpr int MAXK = MK_SAMPLE_MAX_TOPK;

struct SParams {
  const float* logits;
  const float* params;   // [batch][3]: top_k, top_p, temperature
  const int32_t* counter;
  int32_t* tokens;
  float* uniforms;
  unsigned long long seed;
  int vocab, stride;
};

// Order-preserving key of an fp32 value (larger float -> larger key); NaN -> 0.
__device__ __forceinline__ uint32_t okey(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_to_float(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11): 10 rounds of
// (hi, lo) = M * c products mixed with the key, key bumped by the Weyl
// constants between rounds. Returns the first output word.
__device__ __forceinline__ uint32_t philox_first(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0,
                                                 uint32_t k1) {
  constexpr uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u, W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = (uint64_t)M0 * c0, p1 = (uint64_t)M1 * c2;
    const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0, hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
    k0 += W0;
    k1 += W1;
  }
  return c0;
}

struct SLds {
  uint32_t hist[256];
  unsigned long long cand[CAND];   // (key << 32) | (0xffffffff - index): one descending sort
  float csum[CAND];                // inclusive prefix sums of the softmax numerators
  float wsum[ST / 64];
  unsigned long long best[ST / 64];
  uint32_t prefix, need, ncand;
  int nkeep, pick;
};

// Inclusive prefix sum of CAND floats in LDS (Hillis-Steele, fixed order).
__device__ void prefix_sum(float* a) {
  for (int off = 1; off < CAND; off <<= 1) {
    float v[CAND / ST];
#pragma unroll
    for (int j = 0; j < CAND / ST; ++j) {
      const int i = threadIdx.x + j * ST;
      v[j] = i >= off ? a[i - off] : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < CAND / ST; ++j) a[threadIdx.x + j * ST] += v[j];
    __syncthreads();
  }
}

__global__ void __launch_bounds__(ST) mk_sample_kernel(SParams p) {
  __shared__ SLds L;
  const int row = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const float* x = p.logits + (size_t)row * p.stride;
  const float pk = p.params[row * 3 + 0], pp = p.params[row * 3 + 1], temp = p.params[row * 3 + 2];
  const int V = p.vocab;
  int k = (int)pk;

  if (k == 1 || !(temp > 0.f)) {   // greedy: argmax, lowest index on ties
    unsigned long long b = 0xffffffffull;   // key 0 (NaN), index 0
    for (int i = t; i < V; i += ST) {
      const unsigned long long kv = ((unsigned long long)okey(x[i]) << 32) | (0xffffffffu - (uint32_t)i);
      b = kv > b ? kv : b;
    }
    for (int o = 32; o >= 1; o >>= 1) {
      const unsigned long long v = __shfl_xor(b, o, 64);
      b = v > b ? v : b;
    }
    if (lane == 0) L.best[wave] = b;
    __syncthreads();
    if (t == 0) {
      unsigned long long m = L.best[0];
      for (int w = 1; w < ST / 64; ++w) m = L.best[w] > m ? L.best[w] : m;
      p.tokens[row] = (int32_t)(0xffffffffu - (uint32_t)(m & 0xffffffffull));
      if (p.uniforms) p.uniforms[row] = -1.f;
    }
    return;
  }
  if (k <= 0 || k > MAXK) k = MAXK;
  if (k > V) k = V;

  // 1. radix select of the k-th largest key
  if (t == 0) {
    L.prefix = 0u;
    L.need = (uint32_t)k;
    L.ncand = 0u;
  }
  uint32_t mask = 0u;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = t; i < 256; i += ST) L.hist[i] = 0u;
    __syncthreads();
    const uint32_t prefix = L.prefix;
    for (int i = t; i < V; i += ST) {
      const uint32_t kx = okey(x[i]);
      if ((kx & mask) == prefix) atomicAdd(&L.hist[(kx >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (t == 0) {
      uint32_t cum = 0u, need = L.need;
      int d = 255;
      for (; d > 0; --d) {
        if (cum + L.hist[d] >= need) break;
        cum += L.hist[d];
      }
      L.need = need - cum;
      L.prefix = prefix | ((uint32_t)d << shift);
    }
    mask |= 255u << shift;
    __syncthreads();
  }
  const uint32_t thr = L.prefix;   // key of the k-th largest logit

  // 2. gather the tokens at or above it, sort descending (key, then ascending index)
  for (int i = t; i < CAND; i += ST) L.cand[i] = 0ull;
  __syncthreads();
  for (int i = t; i < V; i += ST) {
    const uint32_t kx = okey(x[i]);
    if (kx >= thr) {
      const uint32_t slot = atomicAdd(&L.ncand, 1u);
      if (slot < (uint32_t)CAND) L.cand[slot] = ((unsigned long long)kx << 32) | (0xffffffffu - (uint32_t)i);
    }
  }
  __syncthreads();
  for (int size = 2; size <= CAND; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = t; i < CAND / 2; i += ST) {
        const int lo = 2 * i - (i & (stride - 1)), hi = lo + stride;
        const bool desc = (lo & size) == 0;
        const unsigned long long a = L.cand[lo], b = L.cand[hi];
        if ((a < b) == desc) {
          L.cand[lo] = b;
          L.cand[hi] = a;
        }
      }
      __syncthreads();
    }
  }
  const int n = L.ncand < (uint32_t)CAND ? (int)L.ncand : CAND;

  // 3. softmax numerators in sorted order, prefix sums, nucleus cut, draw
  const float m = key_to_float((uint32_t)(L.cand[0] >> 32)) / temp;
  for (int i = t; i < CAND; i += ST)
    L.csum[i] = i < n ? __expf(key_to_float((uint32_t)(L.cand[i] >> 32)) / temp - m) : 0.f;
  __syncthreads();
  prefix_sum(L.csum);
  const float Z = L.csum[n - 1];
  // kept: position 0, and j >= 1 while csum[j-1] < top_p * Z
  const float cut = (pp > 0.f && pp < 1.f) ? pp * Z : 2.f * Z;
  if (t == 0) L.nkeep = 0;
  __syncthreads();
  int mine = 0;
  for (int j = t; j < n; j += ST) mine += (j == 0 || L.csum[j - 1] < cut) ? 1 : 0;
  atomicAdd(&L.nkeep, mine);
  __syncthreads();
  const int nkeep = L.nkeep;
  const uint32_t c = p.counter ? (uint32_t)p.counter[row] : 0u;
  const uint32_t w = philox_first(c, (uint32_t)row, 0u, 0u, (uint32_t)p.seed, (uint32_t)(p.seed >> 32));
  const float u = (float)(w >> 8) * (1.0f / 16777216.0f);
  const float target = u * L.csum[nkeep - 1];
  if (t == 0) L.pick = nkeep - 1;   // target at the very top (rounding): the last kept token
  __syncthreads();
  // the first j with csum[j] > target: csum is nondecreasing, so exactly one j has
  // csum[j] > target >= csum[j-1]
  for (int j = t; j < nkeep; j += ST)
    if (L.csum[j] > target && (j == 0 || !(L.csum[j - 1] > target))) L.pick = j;
  __syncthreads();
  if (t == 0) {
    p.tokens[row] = (int32_t)(0xffffffffu - (uint32_t)(L.cand[L.pick] & 0xffffffffull));
    if (p.uniforms) p.uniforms[row] = u;
  }
}

thread_local char s_msg[256] = "";

}  // namespace

extern "C" {

const char* mk_sample_last_error(void) { return s_msg; }

int mk_sample(const mk_sample_args* a) {
  if (!a || !a->logits || !a->params || !a->tokens_out) {
    strcpy(s_msg, "args, logits, params or tokens_out is NULL");
    return MK_ERR_NULL;
  }
  if (a->batch < 1 || a->vocab < 1 || a->vocab_stride < a->vocab) {
    strcpy(s_msg, "batch >= 1, vocab >= 1 and vocab_stride >= vocab required");
    return MK_ERR_SHAPE;
  }
  SParams p;
  p.logits = a->logits;
  p.params = a->params;
  p.counter = a->counter;
  p.tokens = a->tokens_out;
  p.uniforms = a->uniforms_out;
  p.seed = a->seed;
  p.vocab = a->vocab;
  p.stride = a->vocab_stride;
  hipLaunchKernelGGL(mk_sample_kernel, dim3(a->batch), dim3(ST), 0, static_cast<hipStream_t>(a->stream), p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    strncpy(s_msg, hipGetErrorString(e), sizeof(s_msg) - 1);
    return MK_ERR_HIP;
  }
  return MK_OK;
}

}  // extern "C"
