// mk_batch.h — internal interface between the C ABI (mk_decode.hip) and the
// batched decode kernel (mk_batch.hip). Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "mk.h"

namespace mk {

constexpr int BATCH_MAX = 32;       // sequences one batched step serves
constexpr int BATT_MAX_SPLIT = 16;  // KV-length splits per (sequence, kv head)

// Workspace of a batched step (max batch M >= 2), bytes:
//   [0, 256)          control words (exit counter, error bits, epoch), as for batch 1
//   256 + 256*b       u64 argmax key of sequence b (one 256-byte line each)
// Arrival counters of one launch, set*bws_cnt_set(M) into the exchange area's
// uncached counter block (two sets, alternating by epoch; each launch zeroes
// the other set):
//     hand-over counters [MK_MAX_LAYERS][5 hand-overs][N_SUB sub-counters], one 128-byte line each
//     attention-split counters u32 [MK_MAX_LAYERS][M][8 kv heads]
//     down-projection row-group counters u32 [MK_MAX_LAYERS][DN_MAX]
constexpr size_t BWS_KEY0 = 256;
constexpr size_t BWS_KEY_STRIDE = 256;
constexpr int N_HANDOVER = 5;   // per layer: qkv, att, h1, act, h2
constexpr int N_SUB = 32;       // sub-counters per hand-over (arrivals spread over N_SUB lines)
constexpr size_t CNT_LINE = 128;
constexpr size_t HCNT_BYTES = (size_t)MK_MAX_LAYERS * N_HANDOVER * N_SUB * CNT_LINE;
constexpr int DN_MAX = 256;     // row groups of the 2-D down projection (grid / 4) at most
constexpr int DN_KQ = 4;        // K quarters of the 2-D down projection
__host__ __device__ inline size_t bws_cnt0(int M) { return BWS_KEY0 + (size_t)M * BWS_KEY_STRIDE; }
__host__ __device__ inline size_t bws_cnt_set(int M) {
  return HCNT_BYTES + (size_t)MK_MAX_LAYERS * M * MK_N_KV_HEADS * 4 + (size_t)MK_MAX_LAYERS * DN_MAX * 4;
}
__host__ __device__ inline size_t batch_ws_bytes(int M) { return bws_cnt0(M); }
// The two counter sets of a batched launch (2 * bws_cnt_set(M) bytes) live in
// a block of uncached device memory owned by the workspace's exchange area
// (sized for BATCH_MAX, so any block serves any batch).
constexpr size_t BCNT_BLOCK_BYTES = 2 * ((size_t)HCNT_BYTES + (size_t)MK_MAX_LAYERS * BATCH_MAX * MK_N_KV_HEADS * 4 +
                                         (size_t)MK_MAX_LAYERS * DN_MAX * 4);
// Largest batch a workspace of `bytes` serves with the batched layout (< 2: batch-1 layout).
inline int batch_of_ws_bytes(size_t bytes) {
  if (bytes < batch_ws_bytes(2)) return 1;
  int m = 2;
  while (m < BATCH_MAX && batch_ws_bytes(m + 1) <= bytes) ++m;
  return m;
}

// Exchange area of a batched step for up to M sequences (bytes), ordinary
// device memory. Two kinds of buffers:
//
// Written once per launch and read only after an arrival counter is complete
// (per layer, each part on a 256-byte boundary), through the XCD's L2:
//   att  bf16 [M16][2048] merged attention output, M16 = M rounded up to 16,
//                         in MFMA A-tile order (1 KiB per 16 tokens x 32 columns)
//   h1   bf16 [M][2048]   h + attn
//   act  bf16 [M16][8192] silu(gate) * up, in A-tile order
//   h2   bf16 [M][2048]   layer output
// then, after all layers, the attention partials
//   part fp32 [layer][M][8 kv][BATT_MAX_SPLIT][m(4) l(4) o(4x64)]
// and the down-projection partials of the four K quarters
//   dpart fp32 [layer][4][M][2048].
//
// Sentinel-filled, in two sets that alternate between launches (the epoch
// picks the set; a launch refills the other one): bytes 0xffff until
// written, so an attention item polls its own token's q and fresh K/V rows
// instead of waiting for every workgroup's QKV stores (per layer):
//   qkv  bf16 [M][3072]   q | fresh k | fresh v of each token
struct BatchLayout {
  size_t att, h1, act, h2, layer;               // write-once region, within a layer
  size_t part_base, part_layer, dpart_base, dpart_layer;
  size_t sq_qkv, sset_layer;                    // sentinel region, within a layer of a set
  size_t sent_base, sset, total;                // sets at sent_base and sent_base + sset
  static constexpr size_t r256(size_t x) { return (x + 255) / 256 * 256; }
  void init(int M) {
    const size_t M16 = (size_t)(M + 15) / 16 * 16;
    att = 0;
    h1 = r256(att + M16 * MK_HIDDEN * 2);
    act = r256(h1 + (size_t)M * MK_HIDDEN * 2);
    h2 = r256(act + M16 * MK_INTER * 2);
    layer = r256(h2 + (size_t)M * MK_HIDDEN * 2);
    part_base = (size_t)MK_MAX_LAYERS * layer;
    part_layer = r256((size_t)M * MK_N_KV_HEADS * BATT_MAX_SPLIT * 4 * (MK_HEAD_DIM + 2) * 4);
    dpart_base = part_base + (size_t)MK_MAX_LAYERS * part_layer;
    dpart_layer = r256((size_t)DN_KQ * M * MK_HIDDEN * 4);
    sq_qkv = 0;
    sset_layer = r256(sq_qkv + (size_t)M * MK_QKV_ROWS * 2);
    sset = (size_t)MK_MAX_LAYERS * sset_layer;
    sent_base = r256(dpart_base + (size_t)MK_MAX_LAYERS * dpart_layer);
    total = sent_base + 2 * sset;
  }
};

// The two-token-tile kernel (batches 17..32) for a grid of `grid` workgroups
// (mk_batch_tile2.hip).
const void* batch_kernel_tile2(int grid);

// Grid check of the batched kernel on a device (occupancy 1 per CU); MK_OK or an MK_ERR code.
int batch_device_check(int dev, char* msg, size_t msg_len);

// Enqueue one batched step (arguments already validated by mk_decode_step):
// xch = exchange area of BatchLayout(max_batch).total bytes, cnt = the two
// zero-initialised counter sets (2 * bws_cnt_set(max_batch) bytes).
hipError_t batch_launch(const mk_weights* w, const mk_step_args* a, uint8_t* xch, uint8_t* cnt, int max_batch,
                        int grid, unsigned long long timeout_ticks);

}  // namespace mk
