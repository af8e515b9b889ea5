#pragma once
// Cross-entropy losses (mirrors ops/loss.h of the reference).
#include "ctd/tensor.h"

namespace ctd::ops {

// logits fp32 [N, V], targets int64 [N] -> scalar [1] = mean over rows.
Tensor cross_entropy(const Tensor& logits, const Tensor& targets);
Tensor cross_entropy_impl(const Tensor& logits, const Tensor& targets);

// loss = sum_i mask_i * (-log p_i[t_i]) / sum_i mask_i; throws in backward if
// sum(mask) == 0.
Tensor cross_entropy_masked(const Tensor& logits, const Tensor& targets,
                            const Tensor& loss_mask);
Tensor cross_entropy_masked_impl(const Tensor& logits, const Tensor& targets,
                                 const Tensor& loss_mask);

// cross_entropy_masked(h W^T, targets, loss_mask) for h [N, H], W [V, H] (the
// tied LM head and its loss) without materialising the [N, V] logits: rows go
// through in chunks of at most a few GB of logits, and when h or W needs a
// gradient the chunk's dlogits, dh and dW (for an upstream gradient of 1) are
// formed right there; backward scales them by the upstream gradient.  The
// loss equals cross_entropy_masked's bit for bit; same error on sum(mask) == 0.
// When H and V are multiples of 16, only rows whose mask value is nonzero go
// through the head (listed and counted on the device): masked-out rows add
// nothing to the loss and get dh = 0, as they would if computed.
Tensor linear_cross_entropy_masked(const Tensor& h, const Tensor& w, const Tensor& targets,
                                   const Tensor& loss_mask);
// Rows per chunk of linear_cross_entropy_masked (process-wide); 0 restores the
// automatic choice (about 0.64 GB of logits per chunk).
void set_linear_cross_entropy_chunk_rows(int64_t rows);
// Whether linear_cross_entropy_masked computes only the active rows where it
// can (default true; false runs every row, for comparisons).
void set_linear_cross_entropy_active_rows(bool on);

}  // namespace ctd::ops
