// mk_prefill.h — internal interface between the C ABI (mk_decode.hip) and the
// layer-major prefill kernels (mk_prefill.hip). Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

#include "mk.h"

namespace mk {

// Tokens one pass of the layer loop takes at most: keeps every buffer offset
// of the GEMMs below 2^31 bytes.
constexpr int PREFILL_MAX_CHUNK = 16384;

// Workspace bytes for a chunk of `tokens` tokens (the activations of one
// layer: residual stream, h1, q, normalised input, attention output, act).
size_t prefill_ws_bytes(int tokens);
// Largest chunk (a multiple of 16 tokens) a workspace of `bytes` holds; 0 if none.
int prefill_chunk_cap(size_t bytes);
// Enqueue the prefill of mk_prefill_args (validated by mk_prefill) in chunks of `cap` tokens.
hipError_t prefill_launch(const mk_weights* w, const mk_prefill_args* a, int cap);

}  // namespace mk
