// fgpt_spec.hip -- host side of greedy speculative decoding: the accept
// rule and the prompt-lookup drafter, as C-ABI functions. No device code;
// the device-resident loop (kern_core.hip k_spec_draft / k_spec_commit,
// fgpt_engine.hip fg_decode_spec) follows the same rules.
//
// The rule is temperature 0 only, as in the reference: the committed
// stream is exactly the target's greedy stream.
#include <cstdint>

#include "../../include/fgpt.h"
#include "fgpt_internal.h"

namespace fgpt {

// accept_prefix (src/lib/fortran_spec.f90:41-52): the longest prefix of
// draft[0:k] that matches targ, and the target id right after it.
int spec_accept_prefix(const int32_t* draft, const int32_t* targ, int k, int32_t* correction) {
  int n = 0;
  while (n < k && draft[n] == targ[n]) ++n;
  *correction = targ[n];
  return n;
}

// lookup_draft (src/lib/fortran_spec.f90:62-92). p = number of known ids
// (ids[0:p]); the last mm = min(m, p-1) ids are searched for in earlier
// windows ending at 1-based position s = p-mm down to mm, the most recent
// first; a hit proposes what followed it, at most k ids and never past p.
int spec_lookup_draft(const int32_t* ids, int p, int m, int k, int32_t* d) {
  const int mm = m < p - 1 ? m : p - 1;
  if (mm < 1) return 0;
  const int32_t* tail = ids + (p - mm);
  for (int s = p - mm; s >= mm; --s) {
    const int32_t* win = ids + (s - mm);
    int j = 0;
    while (j < mm && win[j] == tail[j]) ++j;
    if (j < mm) continue;
    const int kk = k < p - s ? k : p - s;
    for (int i = 0; i < kk; ++i) d[i] = ids[s + i];
    return kk;
  }
  return 0;
}

}  // namespace fgpt

extern "C" int32_t fg_spec_accept(const int32_t* draft, const int32_t* targmax, int32_t k,
                                  int32_t* n_accept, int32_t* correction) {
  if (!targmax || !n_accept || !correction || k < 0 || (k > 0 && !draft))
    return fgpt::set_error(FG_EARG, "fg_spec_accept: bad argument");
  *n_accept = fgpt::spec_accept_prefix(draft, targmax, k, correction);
  return FG_OK;
}

extern "C" int32_t fg_spec_draft(const int32_t* ids, int32_t p, int32_t m, int32_t k,
                                 int32_t* draft, int32_t* n_draft) {
  if (!n_draft || (p > 0 && !ids) || p < 0 || k < 0 || (k > 0 && !draft))
    return fgpt::set_error(FG_EARG, "fg_spec_draft: bad argument");
  *n_draft = fgpt::spec_lookup_draft(ids, p, m, k, draft);
  return FG_OK;
}
