// mk_batch_tile2.hip — the batched decode kernel's two-token-tile
// instantiations (batches 17..32) as a translation unit of their own: the
// kernel source of mk_batch.hip compiled with the thread index opaque to the
// optimiser (MK_BATCH_TILE2; see tid() in mk_common.h). mk_batch.hip's
// batch_kernel_for() hands these out for batches above 16.
#define MK_BATCH_TILE2 1
#include "mk_batch.hip"
