// pbx_spec.cpp -- greedy speculative decoding over two resident models.
//
// The control flow of SelfSpeculativeDecoder.generate (speculative.js:58-204)
// with greedy selection: prefill, then rounds of draft -> verify ->
// accept/reject -> cache rollback.  Two changes of substance, both about
// where the work runs rather than what it computes:
//   * the draft is a separate model with its own KV cache (the reference
//     drafts with the target's first layers, speculative.js:100-102); the
//     draft's greedy chain runs as one pbx_model_generate call (the argmax
//     feeds the next step on the device);
//   * with batched_verify the round's inputs [next, d1..dk] are verified in
//     ONE forward of k+1 rows (pbx_model_forward_batch), whose row i logits
//     are those of the reference's i-th single-token verify forward
//     (speculative.js:131-137) and whose last row is the reference's bonus
//     forward (speculative.js:170-174).

#include <chrono>
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
                    "pbx_speculative_generate: the draft needs its own model (own KV cache)");
  if (!prompt || n_prompt <= 0 || max_tokens <= 0 || !out_tokens || !n_out)
    return pbx_fail(c, PBX_EINVAL, "pbx_speculative_generate: bad arguments");
  if (draft_count < 1 || draft_count > 16)
    return pbx_fail(c, PBX_EINVAL, "pbx_speculative_generate: draft_count %d outside 1..16",
                    draft_count);
  if (n_eos < 0 || (n_eos > 0 && !eos_ids))
    return pbx_fail(c, PBX_EINVAL, "pbx_speculative_generate: bad eos list");
  // Positions reach n_prompt + max_tokens + draft_count in the worst case.
  const int64_t need = (int64_t)n_prompt + max_tokens + draft_count + 1;
  if (need > tc->max_seq || need > dc->max_seq)
    return pbx_fail(c, PBX_EINVAL,
                    "pbx_speculative_generate: %lld positions exceed max_seq (%d target, %d draft)",
                    (long long)need, tc->max_seq, dc->max_seq);
  for (int i = 0; i < n_prompt; ++i)
    if (prompt[i] < 0)
      return pbx_fail(c, PBX_EINVAL, "pbx_speculative_generate: negative prompt token");
  *n_out = 0;
  const int tv = tc->vocab_size, dv = dc->vocab_size;
  int rc;
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
  int dpos = n_prompt;  // draft cache holds positions [0, dpos)
  int pos = n_prompt;
  all.push_back(next);
  int generated = 1;
  bool hit_eos = is_eos(next, eos_ids, n_eos);
  pbx_spec_stats st{};
  std::vector<int32_t> drafts(draft_count), rows(draft_count + 1), preds(draft_count + 1);

  const double t2 = now_ms();
  while (generated < max_tokens && !hit_eos) {
    // Bring the draft's cache up to `pos` (after a fully accepted round the
    // last draft token was never fed to the draft model).
    while (dpos < pos) {
      const int32_t t = to_vocab(all[dpos], dv);
      if ((rc = pbx_model_forward(draft, &t, 1, dpos, nullptr, nullptr))) return rc;
      ++dpos;
    }
    // Draft phase (speculative.js:92-114): up to draft_count greedy tokens,
    // stopping after an EOS draft and at the token budget.
    int k = std::min(draft_count, max_tokens - generated);
    if (is_eos(next, eos_ids, n_eos)) k = 0;
    if (k == 0) break;
    if ((rc = pbx_model_generate(draft, to_vocab(next, dv), pos, k, drafts.data(), nullptr)))
      return rc;
    dpos = pos + k;
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
      // Rows past the accepted prefix were written by this forward: clear
      // them, leaving the cache as the reference's rollbackCache does.
      const int new_pos = bonus ? pos + nd + 1 : pos + accepted + 1;
      if ((rc = pbx_model_clear_range(target, new_pos, pos + nd + 1))) return rc;
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
    if (bonus) {
      pos += nd + 1;
    } else {
      pos += accepted + 1;
      // the draft's cache is valid up to the last accepted draft input
      dpos = std::min(dpos, pos);
    }
    next = all.back();
    st.accepted += accepted;
  }
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
