// The four-wave, two-columns-per-wave prefill kernel (prefill_wide.hip),
// launched by the varlen prefill entry points in prefill.hip.
#pragma once

#include "prefill_common.h"

namespace aac {

// Shapes the wide kernel serves: bf16, GQA groups 2, 4, 8, a positive scale.
bool prefill_wide_supports(int g, float scale, bool f16);

// Launch on the persistent grid (min(items, n_cu) workgroups).  a.n_qblocks
// is set by the launcher.  store: also write the K/V rows to the KV cache
// through a.slots (causal self-attention only).
int prefill_wide_launch(const pf::Args& a, int g, bool causal, bool store, int max_q, int n_cu,
                        hipStream_t st);

}  // namespace aac
