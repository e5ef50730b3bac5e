// Test-only driver around the reference's own host sampler
// (tools/sample/sampler.h, header-only, compiled from where it lies in the
// reference tree into oracle/_ref/).  sample_token() with temp = 1, top_p = 1
// and top_k = k returns, in probs_out, the softmax renormalised over the
// top-k set chosen with the reference's tie rule (sampler.h:90-112).  That is
// the router's softmax -> top-k -> renormalise, so its support pins the
// selected expert set and its values pin the weights.
#include <vector>

#include "sampler.h"

extern "C" int ref_topk_probs(const float *logits, int V, int k,
                              float *probs_out) {
  SampleParams p;
  p.temp = 1.0f;
  p.top_k = k;
  p.top_p = 1.0f;
  p.rep_penalty = 1.0f;
  p.seed = 0;
  uint64_t rng = 1;
  std::vector<float> probs;
  int tok = sample_token(logits, V, p, rng, &probs);
  for (int i = 0; i < V; ++i) probs_out[i] = probs[i];
  return tok;
}
