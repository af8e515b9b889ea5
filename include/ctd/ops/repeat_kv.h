#pragma once
// GQA KV-head expansion and scalar multiply (mirrors ops/repeat_kv.h of the reference).
#include "ctd/tensor.h"

namespace ctd::ops {

// [B, T, H_kv, D] -> [B, T, H_kv*group, D]; backward sums each group.
Tensor repeat_kv_heads(const Tensor& x, int group);
Tensor repeat_kv_heads_impl(const Tensor& x, int group);
Tensor repeat_kv_sum_impl(const Tensor& y, int group);

Tensor mul_scalar(const Tensor& x, float c);
Tensor mul_scalar_impl(const Tensor& x, float c);

}  // namespace ctd::ops
