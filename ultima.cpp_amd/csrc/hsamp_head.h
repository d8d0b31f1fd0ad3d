// Launchers shared by the logits producer's sources (hsamp_head.hip: the entry
// point and the F32 / BF16 heads; hsamp_headq.hip: the norm / fold kernel and
// the quantised heads).
#pragma once

#include <hip/hip_runtime.h>

#include "ultima_hsamp.h"

namespace hsamp {

// values / bytes of one block of a quantised head type (0 for others)
int head_block_values(int dtype);
int head_block_bytes(int dtype);
// the final rmsnorm (and the fold, when h->fold_block divides H) of every row
// into h->normed
hipError_t launch_head_prep(const ultima_hsamp_head* h, hipStream_t s);
// the quantised matvec of h->normed into h->logits (with the logit scale)
hipError_t launch_head_quant(const ultima_hsamp_head* h, hipStream_t s);

}  // namespace hsamp
