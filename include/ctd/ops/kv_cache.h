#pragma once
// KV cache read/write ops (mirrors ops/kv_cache.h of the reference).
#include "ctd/tensor.h"

namespace ctd::ops {

// Writes src [B, T, H_kv, D] into cache [B, H_kv, max_seq, D] at rows
// [pos, pos+T), folding the axis permute into the copy.
void write_kv_inplace(Tensor& cache, const Tensor& src, int pos);

// cache[:, :, :valid_len, :] with each KV head repeated `group` times:
// [B, H_kv * group, valid_len, D].
Tensor read_kv_expanded(const Tensor& cache, int valid_len, int group);

}  // namespace ctd::ops
