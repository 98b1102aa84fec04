// Speculative verification on the batched decode path: PromptLookupDrafter::draft
// (src/speculative.rs:71-101), verify_greedy (src/speculative.rs:204-223) and the engine's
// run_groups flattening (src/engine.rs:702-761), where every group is one sequence's held
// token plus its drafts at consecutive positions, all groups verified in shared passes.
#include <algorithm>
#include <cstring>
#include <vector>

#include "common.h"
#include "host/context.h"

namespace pia {
namespace {

int64_t prompt_lookup(const uint32_t* ctx, int64_t n, int64_t k, int64_t min_ngram, int64_t max_ngram,
                      uint32_t* out) {
  if (k == 0 || n <= min_ngram) return 0;
  const int64_t max_n = std::min(std::max(max_ngram, min_ngram), n - 1);
  // Longest suffix first; within one length the most recent earlier occurrence wins.
  for (int64_t len = max_n; len >= min_ngram; --len) {
    const uint32_t* suffix = ctx + n - len;
    const int64_t limit = n - len;
    for (int64_t start = limit - 1; start >= 0; --start) {
      if (std::memcmp(ctx + start, suffix, static_cast<size_t>(len) * sizeof(uint32_t)) != 0) continue;
      const int64_t from = start + len;
      if (from >= limit) continue;  // the match runs into the suffix itself
      const int64_t take = std::min(k, limit - from);
      std::memcpy(out, ctx + from, static_cast<size_t>(take) * sizeof(uint32_t));
      return take;
    }
  }
  return 0;
}

// Length of the leading run of drafts the model agreed with.
int64_t accepted_run(const uint32_t* drafts, int64_t n_drafts, const uint32_t* model) {
  int64_t a = 0;
  while (a < n_drafts && drafts[a] == model[a]) ++a;
  return a;
}

}  // namespace
}  // namespace pia

using namespace pia;

extern "C" {

pia_status pia_prompt_lookup_draft(const uint32_t* context, int64_t n, int64_t k, int64_t min_ngram,
                                   int64_t max_ngram, uint32_t* out, int64_t* n_out) {
  PIA_API_BEGIN
  PIA_REQUIRE(n_out && (n == 0 || context) && (k == 0 || out), "null argument");
  PIA_REQUIRE(n >= 0 && k >= 0, "negative length");
  PIA_REQUIRE(min_ngram >= 1, "an n-gram needs at least one token");
  *n_out = prompt_lookup(context, n, k, min_ngram, max_ngram, out);
  PIA_API_END
}

pia_status pia_verify_greedy(const uint32_t* drafts, int64_t n_drafts, const uint32_t* model_argmax,
                             int64_t n_argmax, int64_t* n_accepted, uint32_t* corrected) {
  PIA_API_BEGIN
  PIA_REQUIRE(model_argmax && n_accepted && corrected && (n_drafts == 0 || drafts), "null argument");
  PIA_REQUIRE(n_drafts >= 0 && n_argmax == n_drafts + 1,
              "verification needs one model prediction per draft, plus one more");
  const int64_t a = accepted_run(drafts, n_drafts, model_argmax);
  *n_accepted = a;
  *corrected = model_argmax[a];
  PIA_API_END
}

pia_status pia_model_verify_groups(pia_model* m, const pia_spec_group* groups, int64_t n_groups,
                                   const uint32_t* tokens, const int32_t* tables, int64_t capacity,
                                   uint32_t* predictions, int64_t* n_accepted, uint32_t* corrected, int64_t* passes) {
  PIA_API_BEGIN
  PIA_REQUIRE(m && n_groups >= 0 && (n_groups == 0 || (groups && tokens && tables && predictions)), "null argument");
  PIA_REQUIRE(capacity >= 0, "negative capacity");
  // Flatten: entry j of group g is token tokens[off + j] at position pos + j, on g's table.
  std::vector<uint32_t> flat_tok;
  std::vector<int64_t> flat_pos, flat_toff, flat_tlen;
  for (int64_t g = 0; g < n_groups; ++g) {
    const pia_spec_group& gr = groups[g];
    PIA_REQUIRE(gr.n_tokens >= 1, "a group holds at least its held token");
    PIA_REQUIRE(gr.tokens_off >= 0 && gr.pos >= 0 && gr.table_off >= 0 && gr.table_len >= 0, "negative group field");
    for (int64_t j = 0; j < gr.n_tokens; ++j) {
      flat_tok.push_back(tokens[gr.tokens_off + j]);
      flat_pos.push_back(gr.pos + j);
      flat_toff.push_back(gr.table_off);
      flat_tlen.push_back(gr.table_len);
    }
  }
  const int64_t total = static_cast<int64_t>(flat_tok.size());
  const int64_t chunk = capacity == 0 ? std::max<int64_t>(total, 1) : capacity;
  std::vector<int32_t> am(static_cast<size_t>(total));
  int64_t npass = 0;
  // Splitting a group across passes is safe: a pass runs every layer before the next begins,
  // so a later position always finds the K/V of the earlier ones written.
  for (int64_t s = 0; s < total; s += chunk) {
    const int64_t e = std::min(total, s + chunk);
    pia_status st = pia_model_decode(m, flat_tok.data() + s, flat_pos.data() + s, flat_toff.data() + s,
                                     flat_tlen.data() + s, tables, e - s, nullptr, am.data() + s);
    if (st != PIA_OK) fail(st, pia_last_error());
    ++npass;
  }
  for (int64_t i = 0; i < total; ++i) predictions[i] = static_cast<uint32_t>(am[i]);
  int64_t off = 0;
  for (int64_t g = 0; g < n_groups; ++g) {
    const int64_t n = groups[g].n_tokens;
    const int64_t a = accepted_run(tokens + groups[g].tokens_off + 1, n - 1, predictions + off);
    if (n_accepted) n_accepted[g] = a;
    if (corrected) corrected[g] = predictions[off + a];
    off += n;
  }
  if (passes) *passes = npass;
  PIA_API_END
}

}  // extern "C"
