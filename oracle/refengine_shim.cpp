// C entry point over the reference engine's own accept sampler
// (engine/src/sampling.cpp: probabilities, probabilities_rows with its 8-thread
// pool, sample, reject_sample), compiled from the reference sources into
// oracle/_ref/libds41_refengine.so by `make ref`.
// TEST INFRASTRUCTURE ONLY: tests/ check the library's draft sampling and host
// sampler against it, and bench.py times it as the accept CPU baseline.
#include <cstring>
#include <vector>
#include "ds41/engine.hpp"
#include "ds41/spark.h"

// One accept step the way SpeculativeStep runs it (engine/src/speculation.cpp:116-182):
// draft token k from q_k = probabilities(draft row k) with (step, k, Draft) (argmax when
// T == 0), then p = probabilities_rows(target rows) and reject_sample. Returns 0, or -1
// when the engine throws.
extern "C" int refeng_accept_step(const float *target, const float *draft, int drafts, int vocab,
                                  double temperature, double top_p, uint64_t seed, uint64_t step,
                                  int32_t *draft_tokens, ds41_spark_result *out) {
  try {
    const ds41e::Rng rng{seed};
    std::vector<int> proposals;
    std::vector<ds41e::Distribution> q;
    for (int k = 0; k < drafts; ++k) {
      const std::vector<float> logits(draft + (size_t)k * vocab, draft + (size_t)(k + 1) * vocab);
      int token;
      if (temperature == 0) {
        token = ds41e::argmax(logits);
      } else {
        q.push_back(ds41e::probabilities(logits, temperature, top_p));
        token = ds41e::sample(q.back(), rng, step, (uint32_t)k, ds41e::Purpose::Draft);
      }
      proposals.push_back(token);
      draft_tokens[k] = token;
    }
    std::vector<std::vector<float>> rows;
    for (int k = 0; k <= drafts; ++k) rows.emplace_back(target + (size_t)k * vocab, target + (size_t)(k + 1) * vocab);
    const std::vector<ds41e::Distribution> p = ds41e::probabilities_rows(rows, temperature, top_p);
    const ds41e::Verification v = ds41e::reject_sample(proposals, q, p, rng, step, temperature);
    ds41_spark_result r{};
    for (size_t i = 0; i < v.emitted.size() && i < 6; ++i) r.tokens[i] = v.emitted[i];
    r.emitted = (int)v.emitted.size();
    r.accepted_drafts = (int)v.accepted;
    r.accepted_input_rows = (int)v.accepted_input_rows;
    r.rejected = v.rejected ? 1 : 0;
    *out = r;
    return 0;
  } catch (...) {
    return -1;
  }
}

// The engine's probabilities() of one row (the 8-thread path at top_p == 1, T > 0).
extern "C" int refeng_probabilities(const float *x, int vocab, double temperature, double top_p, double *p) {
  try {
    const ds41e::Distribution d = ds41e::probabilities(std::vector<float>(x, x + vocab), temperature, top_p);
    std::memcpy(p, d.data(), sizeof(double) * d.size());
    return 0;
  } catch (...) {
    return -1;
  }
}
