// mk_decode_step.hip — the batch-1 decode kernel's single-step instantiations
// (mk_decode_step, mk_layer_step, mk_decode_step_noalloc) as a translation
// unit of their own: the kernel source of mk_decode.hip compiled with the
// thread index opaque to the optimiser (MK_DECODE_STEP_TU; see tid() in
// mk_common.h). mk_decode.hip's decode_kernel_for() hands these out.
#define MK_DECODE_STEP_TU 1
#include "mk_decode.hip"
