// The reference's src/reference.hpp under its own name, so that its callers (tests/cpu_tests.cpp
// includes "reference.hpp") compile against the drop-in unchanged: the shapes, the paged layout and
// the cache writers of kvb/layout.hpp, plus the declaration of the fp64 attention reference.
#pragma once

#include <span>

#include "kvb/layout.hpp"

namespace kvb {

// out[b][h][d] = softmax_t(scale * q.k_t) . v_t over the contiguous cache [B][Hkv][max_len][D], in
// fp64 with a two-pass softmax; an empty sequence gives 0 (src/reference.hpp:84-89, defined in
// src/reference.cpp:65-100 for T = float and half_t).
//
// Declared only. This build's libraries neither define nor call it: the definition is the
// reference's own CPU code (its `kvref` library, src/reference.cpp), which a caller that uses it links
// beside libkvb_host and libkvb_hip. That is how the reference's test programs and the benchmark's
// CPU rows get their fp64 ground truth; no GPU path depends on it.
template <class T>
void attention_reference(const Shape& s, std::span<const int> seq_lens, int max_len, const float* q, const T* k,
                         const T* v, float* out, float scale, int threads = 1);

}  // namespace kvb
