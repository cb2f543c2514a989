// pbx_spec.cpp -- greedy speculative decoding on resident models.
//
// The control flow of SelfSpeculativeDecoder.generate (speculative.js:58-204)
// with greedy selection: prefill, then rounds of draft -> verify ->
// accept/reject -> cache rollback.  Two drafting modes:
//   * self draft (pbx_self_speculative_generate): the reference's own
//     scheme, the target's first draft_layers layers (forward with
//     {maxLayers}, speculative.js:96-111), replayed as one on-device chain
//     of partial decode steps;
//   * a separate draft model with its own KV cache
//     (pbx_speculative_generate), whose greedy chain runs as one
//     pbx_model_generate call.
// With batched_verify the round's inputs [next, d1..dk] are verified in ONE
// forward of k+1 rows (pbx_model_forward_batch), whose row i logits are
// those of the reference's i-th single-token verify forward
// (speculative.js:131-137) and whose last row is the reference's bonus
// forward (speculative.js:170-174); otherwise one forward per draft token,
// as the reference does.

#include <algorithm>
#include <chrono>
#include <functional>
#include <vector>

#include "pbx_internal.h"

namespace {

double now_ms() {
  return std::chrono::duration<double, std::milli>(
             std::chrono::steady_clock::now().time_since_epoch())
      .count();
}

bool is_eos(int32_t t, const int32_t *eos, int n_eos) {
  for (int i = 0; i < n_eos; ++i)
    if (eos[i] == t) return true;
  return false;
}

int32_t to_vocab(int32_t t, int vocab) { return t % vocab; }

// Drafts k tokens after `next` at `pos` into drafts[0..k); returns a status.
using DraftFn = std::function<int(int32_t next, int pos, int k, int32_t *drafts)>;

// Argument checks shared by both entry points.
int check_args(pbx_ctx *c, const char *fn, const int32_t *prompt, int n_prompt, int max_tokens,
               int draft_count, const int32_t *eos_ids, int n_eos, int32_t *out_tokens,
               int *n_out) {
  if (!prompt || n_prompt <= 0 || max_tokens <= 0 || !out_tokens || !n_out)
    return pbx_fail(c, PBX_EINVAL, "%s: bad arguments", fn);
  if (draft_count < 1 || draft_count > 16)
    return pbx_fail(c, PBX_EINVAL, "%s: draft_count %d outside 1..16", fn, draft_count);
  if (n_eos < 0 || (n_eos > 0 && !eos_ids)) return pbx_fail(c, PBX_EINVAL, "%s: bad eos list", fn);
  for (int i = 0; i < n_prompt; ++i)
    if (prompt[i] < 0) return pbx_fail(c, PBX_EINVAL, "%s: negative prompt token", fn);
  return PBX_OK;
}

// The decode loop after the prefill (speculative.js:85-185) on `target`,
// drafting through `draft`.  `all` holds the prompt and the first token;
// on return it holds every generated token.  draft_written(pos) reports
// the positions past `pos` the draft phase wrote into the target's cache
// (self draft), which the round clears as the reference's rollbackCache
// does.
int spec_loop(pbx_model *target, const DraftFn &draft, bool self_draft, int max_tokens,
              int draft_count, const int32_t *eos_ids, int n_eos, int batched_verify,
              std::vector<int32_t> &all, int pos, pbx_spec_stats &st) {
  const int tv = pbx_model_cfg(target)->vocab_size;
  int32_t next = all.back();
  int generated = 1;
  bool hit_eos = is_eos(next, eos_ids, n_eos);
  std::vector<int32_t> drafts(draft_count), rows(draft_count + 1), preds(draft_count + 1);
  int rc;
  while (generated < max_tokens && !hit_eos) {
    // Draft phase (speculative.js:92-114): up to draft_count greedy tokens,
    // stopping after an EOS draft and at the token budget.
    const int k = std::min(draft_count, max_tokens - generated);
    if (k <= 0) break;
    if ((rc = draft(next, pos, k, drafts.data()))) return rc;
    int nd = 0;
    for (int d = 0; d < k; ++d) {
      drafts[d] = to_vocab(drafts[d], tv);
      ++nd;
      if (is_eos(drafts[d], eos_ids, n_eos)) break;
    }
    st.drafted += nd;
    st.rounds++;

    // Verify phase (speculative.js:120-185).
    rows[0] = next;
    for (int d = 0; d < nd; ++d) rows[d + 1] = drafts[d];
    int accepted = 0;
    bool bonus = false;
    if (batched_verify) {
      if ((rc = pbx_model_forward_batch(target, rows.data(), nd + 1, pos, nullptr, preds.data())))
        return rc;
      for (int d = 0; d < nd; ++d) {
        const int32_t pred = preds[d];
        all.push_back(pred);
        ++generated;
        if (pred == rows[d + 1]) {
          ++accepted;
          if (is_eos(pred, eos_ids, n_eos)) { hit_eos = true; break; }
        } else {
          if (is_eos(pred, eos_ids, n_eos)) hit_eos = true;
          break;
        }
      }
      if (accepted == nd && !hit_eos) {
        const int32_t b = preds[nd];
        all.push_back(b);
        ++generated;
        if (is_eos(b, eos_ids, n_eos)) hit_eos = true;
        bonus = true;
      }
      // Rows past the accepted prefix were written by this forward (and, with
      // the self draft, by the draft's partial steps): clear them, leaving
      // the cache as the reference's rollbackCache does.
      const int new_pos = bonus ? pos + nd + 1 : pos + accepted + 1;
      const int written = self_draft ? std::max(pos + nd + 1, pos + k) : pos + nd + 1;
      if ((rc = pbx_model_clear_range(target, new_pos, written))) return rc;
    } else {
      if ((rc = pbx_model_rollback(target, pos))) return rc;
      for (int d = 0; d < nd; ++d) {
        int32_t pred = 0;
        if ((rc = pbx_model_forward(target, &rows[d], 1, pos + d, nullptr, &pred))) return rc;
        all.push_back(pred);
        ++generated;
        if (pred == rows[d + 1]) {
          ++accepted;
          if (is_eos(pred, eos_ids, n_eos)) { hit_eos = true; break; }
        } else {
          if (is_eos(pred, eos_ids, n_eos)) hit_eos = true;
          if ((rc = pbx_model_rollback(target, pos + d + 2))) return rc;
          break;
        }
      }
      if (accepted == nd && !hit_eos) {
        int32_t b = 0;
        if ((rc = pbx_model_forward(target, &rows[nd], 1, pos + nd, nullptr, &b))) return rc;
        all.push_back(b);
        ++generated;
        if (is_eos(b, eos_ids, n_eos)) hit_eos = true;
        bonus = true;
      }
    }
    pos += bonus ? nd + 1 : accepted + 1;
    next = all.back();
    st.accepted += accepted;
  }
  return PBX_OK;
}

}  // namespace

extern "C" int pbx_speculative_generate(pbx_model *target, pbx_model *draft,
                                        const int32_t *prompt, int n_prompt, int max_tokens,
                                        int draft_count, const int32_t *eos_ids, int n_eos,
                                        int batched_verify, int32_t *out_tokens, int *n_out,
                                        pbx_spec_stats *stats) {
  const pbx_model_config *tc = pbx_model_cfg(target), *dc = pbx_model_cfg(draft);
  if (!tc || !dc)
    return pbx_fail(tc ? pbx_model_ctx(target) : nullptr, PBX_EINVAL,
                    "pbx_speculative_generate: target and draft must be live models");
  pbx_ctx *c = pbx_model_ctx(target);
  if (pbx_model_ctx(draft) != c)
    return pbx_fail(c, PBX_EINVAL, "pbx_speculative_generate: models of different contexts");
  if (target == draft)
    return pbx_fail(c, PBX_EINVAL,
                    "pbx_speculative_generate: the draft needs its own model (own KV cache); "
                    "pbx_self_speculative_generate drafts with the target's first layers");
  int rc = check_args(c, "pbx_speculative_generate", prompt, n_prompt, max_tokens, draft_count,
                      eos_ids, n_eos, out_tokens, n_out);
  if (rc) return rc;
  // Positions reach n_prompt + max_tokens + draft_count in the worst case.
  const int64_t need = (int64_t)n_prompt + max_tokens + draft_count + 1;
  if (need > tc->max_seq || need > dc->max_seq)
    return pbx_fail(c, PBX_EINVAL,
                    "pbx_speculative_generate: %lld positions exceed max_seq (%d target, %d draft)",
                    (long long)need, tc->max_seq, dc->max_seq);
  *n_out = 0;
  const int tv = tc->vocab_size, dv = dc->vocab_size;
  if ((rc = pbx_model_reset_cache(target)) || (rc = pbx_model_reset_cache(draft))) return rc;

  // all[p] is the token at position p (prompt, then generated tokens).
  std::vector<int32_t> all(prompt, prompt + n_prompt), tp(n_prompt), dp(n_prompt);
  for (int i = 0; i < n_prompt; ++i) {
    tp[i] = to_vocab(prompt[i], tv);
    dp[i] = to_vocab(prompt[i], dv);
  }
  const double t0 = now_ms();
  int32_t next = 0;
  if ((rc = pbx_model_forward(target, tp.data(), n_prompt, 0, nullptr, &next))) return rc;
  const double t1 = now_ms();
  if ((rc = pbx_model_forward(draft, dp.data(), n_prompt, 0, nullptr, nullptr))) return rc;
  all.push_back(next);
  pbx_spec_stats st{};
  int dpos = n_prompt;  // the draft's cache holds positions [0, dpos)
  DraftFn draft_fn = [&](int32_t nx, int pos, int k, int32_t *out) -> int {
    // the draft's cache is valid up to the last accepted input; bring it up
    // to `pos` (after a fully accepted round the last draft token was never
    // fed to the draft model)
    dpos = std::min(dpos, pos);
    int r;
    while (dpos < pos) {
      const int32_t t = to_vocab(all[dpos], dv);
      if ((r = pbx_model_forward(draft, &t, 1, dpos, nullptr, nullptr))) return r;
      ++dpos;
    }
    if ((r = pbx_model_generate(draft, to_vocab(nx, dv), pos, k, out, nullptr))) return r;
    dpos = pos + k;
    return PBX_OK;
  };
  const double t2 = now_ms();
  if ((rc = spec_loop(target, draft_fn, false, max_tokens, draft_count, eos_ids, n_eos,
                      batched_verify, all, n_prompt, st)))
    return rc;
  if (hipStreamSynchronize(c->stream) != hipSuccess)
    return pbx_fail(c, PBX_EHIP, "pbx_speculative_generate: device failure");
  const double t3 = now_ms();
  const int n = (int)all.size() - n_prompt;
  for (int i = 0; i < n; ++i) out_tokens[i] = all[n_prompt + i];
  *n_out = n;
  st.prefill_ms = t1 - t0;
  st.decode_ms = t3 - t2;
  if (stats) *stats = st;
  return PBX_OK;
}

extern "C" int pbx_self_speculative_generate(pbx_model *m, const int32_t *prompt, int n_prompt,
                                             int max_tokens, int draft_layers, int draft_count,
                                             const int32_t *eos_ids, int n_eos,
                                             int batched_verify, int32_t *out_tokens, int *n_out,
                                             pbx_spec_stats *stats) {
  const pbx_model_config *g = pbx_model_cfg(m);
  if (!g)
    return pbx_fail(nullptr, PBX_EINVAL, "pbx_self_speculative_generate: not a live model");
  pbx_ctx *c = pbx_model_ctx(m);
  int rc = check_args(c, "pbx_self_speculative_generate", prompt, n_prompt, max_tokens,
                      draft_count, eos_ids, n_eos, out_tokens, n_out);
  if (rc) return rc;
  if (draft_layers < 1)
    return pbx_fail(c, PBX_EINVAL, "pbx_self_speculative_generate: draft_layers %d < 1",
                    draft_layers);
  const int64_t need = (int64_t)n_prompt + max_tokens + draft_count + 1;
  if (need > g->max_seq)
    return pbx_fail(c, PBX_EINVAL,
                    "pbx_self_speculative_generate: %lld positions exceed max_seq %d",
                    (long long)need, g->max_seq);
  for (int i = 0; i < n_prompt; ++i)
    if (prompt[i] >= g->vocab_size)
      return pbx_fail(c, PBX_EINVAL, "pbx_self_speculative_generate: token %d out of range",
                      prompt[i]);
  *n_out = 0;
  if ((rc = pbx_model_reset_cache(m))) return rc;
  std::vector<int32_t> all(prompt, prompt + n_prompt);
  const double t0 = now_ms();
  int32_t next = 0;
  if ((rc = pbx_model_forward(m, prompt, n_prompt, 0, nullptr, &next))) return rc;
  const double t1 = now_ms();
  all.push_back(next);
  pbx_spec_stats st{};
  // speculative.js:96-111: forward([t], draftPos, {maxLayers: draftLayers})
  // and argmax, draft_count times, on the target's own cache
  DraftFn draft_fn = [&](int32_t nx, int pos, int k, int32_t *out) -> int {
    return pbx_model_generate_layers(m, nx, pos, k, draft_layers, out);
  };
  if ((rc = spec_loop(m, draft_fn, true, max_tokens, draft_count, eos_ids, n_eos, batched_verify,
                      all, n_prompt, st)))
    return rc;
  if (hipStreamSynchronize(c->stream) != hipSuccess)
    return pbx_fail(c, PBX_EHIP, "pbx_self_speculative_generate: device failure");
  const double t3 = now_ms();
  const int n = (int)all.size() - n_prompt;
  for (int i = 0; i < n; ++i) out_tokens[i] = all[n_prompt + i];
  *n_out = n;
  st.prefill_ms = t1 - t0;
  st.decode_ms = t3 - t1;
  if (stats) *stats = st;
  return PBX_OK;
}
