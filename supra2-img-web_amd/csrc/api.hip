// C ABI of the attention operator and the linear layer: argument validation, kernel selection and
// the device-runtime helpers the JS addon and the Python bindings use.
//
// The operator contract follows app/gpu/ops.js:103-149 (offsets/strides in floats, default output
// row stride H*D, synchronous error for an unsupported request) extended with batch strides, a
// per-sequence key length or boolean key mask, and an in-kernel relative-position bias.

#include <hip/hip_runtime.h>

#include <math.h>
#include <algorithm>
#include <atomic>
#include <mutex>
#include <stddef.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "supra_attn.h"
#include "supra_linear.h"
#include "supra_vae.h"
#include "common.h"
#include "kernels.h"
#include "status.h"

namespace {
thread_local char g_err[sa::kErrorBytes] = "";
thread_local int g_status = SA_OK;
}  // namespace

namespace sa {

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  g_status = code;
  return code;
}

int ok() {
  g_err[0] = '\0';
  g_status = SA_OK;
  return SA_OK;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(SA_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

const char* last_error() { return g_err; }

}  // namespace sa

namespace {

using sa::fail;
using sa::hip_fail;
using sa::ok;

// Byte extent [lo, hi) touched by a strided [B, L, H*D] view of `base`; ok is false when the
// arithmetic overflows (then lo and hi mean nothing).
struct Extent {
  uintptr_t lo, hi;
  bool ok;
};

Extent extent(const void* base, int64_t off, int64_t sb, int64_t ld, int B, int L, int64_t row) {
  int64_t last = off, t = 0;
  bool ok = true;
  if (B > 1) ok = !__builtin_mul_overflow((int64_t)(B - 1), sb, &t) && !__builtin_add_overflow(last, t, &last);
  if (ok && L > 1) ok = !__builtin_mul_overflow((int64_t)(L - 1), ld, &t) && !__builtin_add_overflow(last, t, &last);
  ok = ok && !__builtin_add_overflow(last, row, &last) && last >= 0 && last <= INT64_MAX / 4;
  uintptr_t lo = 0, hi = 0;
  ok = ok && !__builtin_add_overflow((uintptr_t)base, (uintptr_t)off * 4, &lo) &&
       !__builtin_add_overflow((uintptr_t)base, (uintptr_t)last * 4, &hi);
  return {lo, hi, ok};
}

bool overlaps(const Extent& a, const Extent& b) { return a.lo < b.hi && b.lo < a.hi; }

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

// Offsets and strides (in floats) at or above 2^40 (4 TiB) are rejected, so that the extent and
// address arithmetic below stays far from int64 overflow.
constexpr int64_t kMaxExtent = (int64_t)1 << 40;
bool too_large(int64_t v) { return v >= kMaxExtent; }

// Size of the revision-2 struct (it ended at workspace_bytes); still accepted.
constexpr uint32_t kAttnArgsV2Size = offsetof(sa_attn_args, key_len_host);
// Sizes of the revision-1 sa_attn_plan (it ended at tail_workgroups) and of revision 2 (it ended at
// sequence_order); still accepted.
constexpr uint32_t kPlanV1Size = offsetof(sa_attn_plan, order_n);
constexpr uint32_t kPlanV2Size = offsetof(sa_attn_plan, tail_folded);
bool plan_size_ok(uint32_t size) { return size == sizeof(sa_attn_plan) || size == kPlanV2Size || size == kPlanV1Size; }

int num_cus();

// Schedule for per-sequence key lengths known on the host (order[rank] = sequence). The flash
// grid's workgroup remap gives L2 domain (XCD) x the ranks [x*B/8, (x+1)*B/8) in launch order, T
// consecutive units (query tiles x heads) per rank, and within a domain the hardware deals
// workgroup j of the first residency to CU j % C (C CUs per domain, S workgroups per CU: 4 for the
// unbiased head-dim-64 single-split kernel, 1 for the others; the later workgroups take the first
// slots that free up). A CU's time is about the sum of its units' key blocks, so:
//   1. sequences sorted by key blocks, longest first (stable), go to the domain with the least work
//      so far among those not yet full (B/8 each) - the sums per domain come out nearly equal;
//   2. in each domain, from longest first, pairs of positions are swapped while that lowers the
//      heaviest CU's blocks (then the sum of squares) in a simulation of that dealing.
// The model puts the heaviest CU of the batch-64 sweep's cross-attention at 12 blocks (the bound)
// against 13 for dealing longest first round-robin; on the hardware, where later workgroups take
// whichever slot frees first, some CUs still get 13. Measured against the round-robin deal: 34.3 ->
// 33.8 us for the launch, 120.1 -> 118.6 us for a self + cross pair; step 1 alone measured 34.5 us.
//
// Host cost. The search of step 2 is resumable and advances by at most kSearchOpsPerCall simulated
// workgroup placements per call, so a new set of key lengths costs one bounded step (8 us median on
// the build host at batch 64, against 0.5-1.2 ms for the whole search): its first launch runs the
// domain-balanced order of step 1 improved by that step, and each later call with the same lengths
// continues the search from where the last one stopped until it converges (the batch-64 sweep's
// cross-attention after 81 calls; the DiT repeats its prompts in all 14 blocks of every step). The
// whole search is capped at kSearchOps placements; a launch for which one pass over the pairs does
// not fit takes the round-robin deal of the longest-first order, and a B that 8 does not divide
// step 1 alone, over the rank ranges the remap gives each domain (batch 58 of the sweep's lengths:
// 46.6 us for plain longest first, which put every long sequence in the first domains). States are kept for the last kScheduleSlots length sets (a guidance caller
// alternates two), each behind its own mutex: callers with different key lengths never wait for one
// another, and callers with the same lengths wait at most one step.
constexpr int64_t kSearchOps = 1 << 19;
constexpr int64_t kSearchOpsPerCall = 1 << 11;
constexpr int kScheduleSlots = 16;

struct ScheduleModel {
  int B, Lk, C, S;
  int64_t T;
};

int64_t simulate_domain(const uint8_t* seq, int n, const int* nb, int T, int C, int S, int64_t* sumsq) {
  int load[64];
  for (int c = 0; c < C; ++c) load[c] = 0;
  int j = 0, jc = 0;  // jc = j % C (no division in the loop)
  for (int r = 0; r < n; ++r) {
    const int w = nb[seq[r]];
    for (int t = 0; t < T; ++t, ++j) {
      if (j < S * C) {
        load[jc] += w;
        if (++jc == C) jc = 0;
      } else {  // a later workgroup: the slot that frees first, taken as the least loaded CU
        int best = 0, bv = load[0];
        for (int c = 1; c < C; ++c) {  // branch-free (selects): the comparisons are unpredictable
          const bool lt = load[c] < bv;
          bv = lt ? load[c] : bv;
          best = lt ? c : best;
        }
        load[best] += w;
      }
    }
  }
  int64_t mx = 0, sq = 0;
  for (int c = 0; c < C; ++c) {
    mx = std::max<int64_t>(mx, load[c]);
    sq += (int64_t)load[c] * load[c];
  }
  *sumsq = sq;
  return mx;
}

// The search of step 2 as a resumable state: domain x, pass, pair (u, v), the domain's current
// heaviest CU and sum of squares, and what it has spent.
struct ScheduleState {
  ScheduleModel m;
  int32_t len[sa::kMaxOrder];
  uint8_t order[sa::kMaxOrder];
  int nb[sa::kMaxOrder];
  int start[9] = {};  // domain x holds the ranks [start[x], start[x + 1])
  int64_t sim_ops = 0;  // of the largest domain
  bool done = true;
  int x = 0, pass = 0, u = 0, v = 0;
  bool dom_started = false, improved = false;
  int64_t mx = 0, sq = 0, spent = 0;
};

// Steps 1 (and the fallbacks) for st.m / st.len: fills st.order and arms the search.
void schedule_start(ScheduleState& st) {
  const ScheduleModel& m = st.m;
  const int B = m.B;
  int idx[sa::kMaxOrder];
  int top = 0;
  for (int i = 0; i < B; ++i) {
    st.nb[i] = (std::min(std::max(st.len[i], 0), m.Lk) + 31) / 32;
    top = std::max(top, st.nb[i]);
  }
  // sequences by key blocks, most first, stable: a counting sort (the comparisons of an insertion
  // sort are unpredictable branches), or a merge sort for very long keys
  constexpr int kBins = 1024;
  if (top < kBins) {
    int start[kBins + 1];
    for (int v = 0; v <= top + 1; ++v) start[v] = 0;
    for (int i = 0; i < B; ++i) ++start[top - st.nb[i] + 1];
    for (int v = 1; v <= top + 1; ++v) start[v] += start[v - 1];
    for (int i = 0; i < B; ++i) idx[start[top - st.nb[i]]++] = i;
  } else {
    for (int i = 0; i < B; ++i) idx[i] = i;
    std::stable_sort(idx, idx + B, [&](int a, int b) { return st.nb[a] > st.nb[b]; });
  }
  st.done = true;
  if (st.nb[idx[0]] == st.nb[idx[B - 1]]) {  // all equal: the launch order, i.e. no schedule
    for (int j = 0; j < B; ++j) st.order[j] = (uint8_t)idx[j];
    return;
  }
  // The remap gives L2 domain x the B*T/8 tiles (to within one) from tile lo_x = x*q + min(x, r) on
  // (q, r = the tile count over 8 and its remainder), i.e. the ranks from about lo_x / T: domain x
  // holds the ranks [start[x], start[x + 1]) with start[x] = lo_x / T rounded (x*B/8 when 8 divides B).
  {
    const int64_t T = std::max<int64_t>(m.T, 1), n = (int64_t)B * T, q = n / 8, r = n % 8;
    for (int x = 0; x < 8; ++x) st.start[x] = (int)((x * q + std::min<int64_t>(x, r) + T / 2) / T);
    st.start[8] = B;
  }
  int most = 0;
  for (int x = 0; x < 8; ++x) most = std::max(most, st.start[x + 1] - st.start[x]);
  // Work of one simulation of the largest domain (workgroups, the later ones scanning C CUs) and of
  // one pass over its pairs in every domain; without room for one pass, 8 dividing B, the
  // round-robin deal.
  const int64_t units = most * std::min<int64_t>(std::max<int64_t>(m.T, 1), 1 << 20);
  const int64_t sim_ops = units + std::max<int64_t>(units - (int64_t)m.S * m.C, 0) * m.C;
  const int64_t pairs = (int64_t)most * (most - 1) / 2;
  const bool search = !(pairs == 0 || m.C < 1 || m.C > 64 || m.T < 1 || m.T > (1 << 20) || 8 * pairs * sim_ops > kSearchOps);
  if (!search && B % 8 == 0) {
    const int per = B / 8;
    for (int j = 0; j < B; ++j) st.order[(j % 8) * per + j / 8] = (uint8_t)idx[j];
    return;
  }
  // step 1: longest first, each sequence to the domain with the least work among those not yet full
  int64_t total[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int count[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int j = 0; j < B; ++j) {
    int best = 0;
    int64_t bv = INT64_MAX;
    for (int x = 0; x < 8; ++x) {  // branch-free: the least work among the domains not yet full
      const bool take = count[x] < st.start[x + 1] - st.start[x] && total[x] < bv;
      bv = take ? total[x] : bv;
      best = take ? x : best;
    }
    st.order[st.start[best] + count[best]++] = (uint8_t)idx[j];
    total[best] += st.nb[idx[j]];
  }
  if (!search) return;
  st.sim_ops = sim_ops;
  st.done = false;
  st.x = 0;
  st.dom_started = false;
}

// Advances the search by at most `budget` simulated placements (one simulation always fits).
void schedule_advance(ScheduleState& st, int64_t budget) {
  const int64_t domain_ops = kSearchOps / 8;
  const int T = (int)st.m.T, C = st.m.C, S = st.m.S;
  while (!st.done && budget > 0) {
    uint8_t* seq = st.order + st.start[st.x];  // longest first within the domain already
    const int per = st.start[st.x + 1] - st.start[st.x];
    if (!st.dom_started) {
      st.mx = simulate_domain(seq, per, st.nb, T, C, S, &st.sq);
      st.spent = st.sim_ops;
      budget -= st.sim_ops;
      st.dom_started = true;
      st.pass = 0;
      st.u = 0;
      st.v = 1;
      st.improved = false;
      continue;
    }
    bool next_domain = st.pass >= 8 || st.spent + st.sim_ops > domain_ops;
    if (!next_domain && st.v >= per) {
      ++st.u;
      st.v = st.u + 1;
    }
    if (!next_domain && st.u >= per - 1) {  // the end of a pass
      if (!st.improved) {
        next_domain = true;
      } else {
        ++st.pass;
        st.u = 0;
        st.v = 1;
        st.improved = false;
        continue;
      }
    }
    if (next_domain) {
      st.dom_started = false;
      if (++st.x == 8) st.done = true;
      continue;
    }
    const int u = st.u, v = st.v++;
    if (st.nb[seq[u]] == st.nb[seq[v]]) continue;
    std::swap(seq[u], seq[v]);
    int64_t sq2;
    const int64_t mx2 = simulate_domain(seq, per, st.nb, T, C, S, &sq2);
    st.spent += st.sim_ops;
    budget -= st.sim_ops;
    if (mx2 < st.mx || (mx2 == st.mx && sq2 < st.sq)) {
      st.mx = mx2;
      st.sq = sq2;
      st.improved = true;
    } else {
      std::swap(seq[u], seq[v]);
    }
  }
}

uint64_t schedule_key(const int32_t* len, const ScheduleModel& m) {
  uint64_t h = 1469598103934665603ull;  // FNV-1a over 32-bit words of the model and the lengths
  auto mix = [&](uint64_t v) {
    h = (h ^ (uint32_t)v) * 1099511628211ull;
    h = (h ^ (uint32_t)(v >> 32)) * 1099511628211ull;
  };
  mix((uint64_t)m.B);
  mix((uint64_t)m.Lk);
  mix((uint64_t)m.C);
  mix((uint64_t)m.S);
  mix((uint64_t)m.T);
  for (int i = 0; i < m.B; ++i) h = (h ^ (uint32_t)len[i]) * 1099511628211ull;
  return h;
}

struct ScheduleSlot {
  std::mutex mu;  // guards st
  ScheduleState st;
};
struct ScheduleCache {
  std::mutex mu;  // guards key / next only (held for a lookup, never during a search step)
  uint64_t key[kScheduleSlots] = {};
  int next = 0;  // slot the next new length set takes
  ScheduleSlot slot[kScheduleSlots];
};
ScheduleCache g_schedule;

bool same_model(const ScheduleModel& a, const ScheduleModel& b) {
  return a.B == b.B && a.Lk == b.Lk && a.C == b.C && a.S == b.S && a.T == b.T;
}

// The order for these lengths: the state of their slot advanced by one bounded step (a new slot is
// started first). Two length sets that share a slot's key, or that race for one slot, restart it:
// the order copied out always belongs to `len`.
void cached_schedule(const int32_t* len, const ScheduleModel& m, uint8_t* order) {
  const uint64_t key = schedule_key(len, m);
  int i = -1;
  {
    std::lock_guard<std::mutex> lock(g_schedule.mu);
    for (int s = 0; s < kScheduleSlots; ++s)
      if (g_schedule.key[s] == key) i = s;
    if (i < 0) {
      i = g_schedule.next;
      g_schedule.next = (g_schedule.next + 1) % kScheduleSlots;
      g_schedule.key[i] = key;
    }
  }
  ScheduleSlot& slot = g_schedule.slot[i];
  std::lock_guard<std::mutex> lock(slot.mu);
  ScheduleState& st = slot.st;
  if (!same_model(st.m, m) || memcmp(st.len, len, (size_t)m.B * sizeof(int32_t)) != 0) {
    st.m = m;
    memcpy(st.len, len, (size_t)m.B * sizeof(int32_t));
    schedule_start(st);
  }
  schedule_advance(st, kSearchOpsPerCall);
  memcpy(order, st.order, (size_t)m.B);
}

// Resolves an sa_attn_args into kernel parameters; returns SA_OK or an error (message set).
int resolve(const sa_attn_args* a, sa::AttnParams* p) {
  if (a == nullptr) return fail(SA_ERR_INVALID, "args is NULL");
  if (a->struct_size != sizeof(sa_attn_args) && a->struct_size != kAttnArgsV2Size)
    return fail(SA_ERR_INVALID, "struct_size %u does not match sizeof(sa_attn_args) = %zu", a->struct_size,
                sizeof(sa_attn_args));
  const int32_t* key_len_host = a->struct_size >= sizeof(sa_attn_args) ? a->key_len_host : nullptr;
  if (a->B < 1 || a->H < 1 || a->D < 1 || a->Lq < 1 || a->Lk < 1)
    return fail(SA_ERR_INVALID, "B, H, D, Lq, Lk must be >= 1 (got B=%d H=%d D=%d Lq=%d Lk=%d)", a->B, a->H, a->D,
                a->Lq, a->Lk);
  if (!a->q || !a->k || !a->v || !a->o) return fail(SA_ERR_INVALID, "q, k, v and o must be non-NULL");
  if (!(isfinite(a->scale))) return fail(SA_ERR_INVALID, "scale must be finite");
  const int64_t HD = (int64_t)a->H * a->D;
  const int64_t ldo = a->ldo > 0 ? a->ldo : HD;
  if (a->q_off < 0 || a->k_off < 0 || a->v_off < 0 || a->o_off < 0)
    return fail(SA_ERR_INVALID, "offsets must be >= 0");
  if (a->ldq < HD || a->ldk < HD || a->ldv < HD || ldo < HD)
    return fail(SA_ERR_INVALID, "row strides must be >= H*D = %lld (ldq=%lld ldk=%lld ldv=%lld ldo=%lld)",
                (long long)HD, (long long)a->ldq, (long long)a->ldk, (long long)a->ldv, (long long)ldo);
  if (a->B > 1 && (a->sq < 0 || a->sk < 0 || a->sv < 0 || a->so < 0))
    return fail(SA_ERR_INVALID, "batch strides must be >= 0");
  if (too_large(a->q_off) || too_large(a->k_off) || too_large(a->v_off) || too_large(a->o_off) ||
      too_large(a->ldq) || too_large(a->ldk) || too_large(a->ldv) || too_large(ldo) || too_large(a->sq) ||
      too_large(a->sk) || too_large(a->sv) || too_large(a->so) || too_large(a->sbias) || too_large(a->smask))
    return fail(SA_ERR_INVALID, "offsets and strides must be below 2^40 elements");
  const int64_t so = a->B > 1 ? a->so : 0;
  if (a->B > 1 && so < (int64_t)(a->Lq - 1) * ldo + HD)
    return fail(SA_ERR_INVALID, "output batch stride %lld makes sequences overlap", (long long)so);

  // o must not overlap q, k or v (WebGPU forbids binding one buffer as read and read_write in one
  // dispatch, so the reference never does this either).
  const Extent eo = extent(a->o, a->o_off, so, ldo, a->B, a->Lq, HD);
  const Extent eq = extent(a->q, a->q_off, a->sq, a->ldq, a->B, a->Lq, HD);
  const Extent ek = extent(a->k, a->k_off, a->sk, a->ldk, a->B, a->Lk, HD);
  const Extent ev = extent(a->v, a->v_off, a->sv, a->ldv, a->B, a->Lk, HD);
  if (!eo.ok || !eq.ok || !ek.ok || !ev.ok)
    return fail(SA_ERR_INVALID, "the extent of q, k, v or o overflows 64-bit addresses");
  if (overlaps(eo, eq) || overlaps(eo, ek) || overlaps(eo, ev))
    return fail(SA_ERR_ALIAS, "the output overlaps q, k or v");

  // The other operands the kernels read (bias, bucket LUT, key lengths, key mask) must not overlap
  // the output either: other workgroups write o while they are read.
  auto span = [](const void* base, int64_t off_bytes, int64_t bytes) -> Extent {
    uintptr_t lo = 0, hi = 0;
    const bool ok = off_bytes >= 0 && bytes >= 0 && !__builtin_add_overflow((uintptr_t)base, (uintptr_t)off_bytes, &lo) &&
                    !__builtin_add_overflow(lo, (uintptr_t)bytes, &hi);
    return {lo, hi, ok};
  };
  switch (a->bias_mode) {
    case SA_BIAS_NONE:
      break;
    case SA_BIAS_DENSE: {
      if (!a->bias) return fail(SA_ERR_INVALID, "SA_BIAS_DENSE needs bias");
      if (a->B > 1 && a->sbias < 0) return fail(SA_ERR_INVALID, "sbias must be >= 0");
      const Extent eb = extent(a->bias, 0, a->sbias, 0, a->B, 1, (int64_t)a->H * a->Lq * a->Lk);
      if (!eb.ok) return fail(SA_ERR_INVALID, "the extent of the dense bias overflows 64-bit addresses");
      if (overlaps(eo, eb)) return fail(SA_ERR_ALIAS, "the output overlaps the dense bias");
      break;
    }
    case SA_BIAS_RELPOS: {
      if (!a->bias || !a->bucket_lut) return fail(SA_ERR_INVALID, "SA_BIAS_RELPOS needs bias (table) and bucket_lut");
      if (a->num_buckets < 1) return fail(SA_ERR_INVALID, "SA_BIAS_RELPOS needs num_buckets >= 1");
      const Extent et = span(a->bias, 0, (int64_t)a->num_buckets * a->H * 4);
      const Extent el = span(a->bucket_lut, 0, ((int64_t)a->Lq + a->Lk - 1) * 4);
      if (overlaps(eo, et) || overlaps(eo, el))
        return fail(SA_ERR_ALIAS, "the output overlaps the relative-position table or bucket LUT");
      break;
    }
    default:
      return fail(SA_ERR_INVALID, "unknown bias_mode %d", a->bias_mode);
  }
  switch (a->mask_mode) {
    case SA_MASK_NONE:
      break;
    case SA_MASK_KEY_LEN:
      if (!a->key_len) return fail(SA_ERR_INVALID, "SA_MASK_KEY_LEN needs key_len");
      if (overlaps(eo, span(a->key_len, 0, (int64_t)a->B * 4)))
        return fail(SA_ERR_ALIAS, "the output overlaps key_len");
      break;
    case SA_MASK_KEY_MASK: {
      if (!a->key_mask) return fail(SA_ERR_INVALID, "SA_MASK_KEY_MASK needs key_mask");
      if (a->B > 1 && a->smask > 0 && a->smask < a->Lk)
        return fail(SA_ERR_INVALID, "smask %lld is smaller than Lk", (long long)a->smask);
      const int64_t sm = a->smask > 0 ? a->smask : a->Lk;
      if (overlaps(eo, span(a->key_mask, 0, (int64_t)(a->B - 1) * sm + a->Lk)))
        return fail(SA_ERR_ALIAS, "the output overlaps key_mask");
      break;
    }
    default:
      return fail(SA_ERR_INVALID, "unknown mask_mode %d", a->mask_mode);
  }

  p->q = a->q;
  p->k = a->k;
  p->v = a->v;
  p->o = a->o;
  p->q_off = a->q_off;
  p->k_off = a->k_off;
  p->v_off = a->v_off;
  p->o_off = a->o_off;
  p->ldq = a->ldq;
  p->ldk = a->ldk;
  p->ldv = a->ldv;
  p->ldo = ldo;
  p->sq = a->B > 1 ? a->sq : 0;
  p->sk = a->B > 1 ? a->sk : 0;
  p->sv = a->B > 1 ? a->sv : 0;
  p->so = so;
  p->B = a->B;
  p->H = a->H;
  p->D = a->D;
  p->Lq = a->Lq;
  p->Lk = a->Lk;
  p->scale_log2 = a->scale * sa::kLog2e;
  p->bias_mode = a->bias_mode;
  p->bias = a->bias;
  p->sbias = a->B > 1 ? a->sbias : 0;
  p->lut = a->bucket_lut;
  p->num_buckets = a->num_buckets;
  p->mask_mode = a->mask_mode;
  p->key_len = a->key_len;
  p->key_mask = a->key_mask;
  p->smask = a->B > 1 ? (a->smask > 0 ? a->smask : a->Lk) : 0;
  // the sequence schedule, if any, is made for the chosen kernel (apply_schedule)
  p->key_len_host = a->mask_mode == SA_MASK_KEY_LEN ? key_len_host : nullptr;
  p->order_n = 0;
  return SA_OK;
}

// Resolves an sa_linear_args (app/gpu/ops.js:35-43 semantics) into kernel parameters.
int resolve_linear(const sa_linear_args* a, sa::LinearParams* p) {
  if (a == nullptr) return fail(SA_ERR_INVALID, "args is NULL");
  if (a->struct_size != sizeof(sa_linear_args))
    return fail(SA_ERR_INVALID, "struct_size %u does not match sizeof(sa_linear_args) = %zu", a->struct_size,
                sizeof(sa_linear_args));
  if (a->M <= 0 || a->N <= 0 || a->K <= 0)
    return fail(SA_ERR_INVALID, "M, N, K must be positive (got %d, %d, %d)", a->M, a->N, a->K);
  if (!a->x || !a->w || !a->y) return fail(SA_ERR_INVALID, "x, w and y must be non-NULL device pointers");
  if (a->x_off < 0 || a->y_off < 0 || a->gate_off < 0) return fail(SA_ERR_INVALID, "offsets must be >= 0");
  const int64_t ldx = a->ldx ? a->ldx : a->K, ldw = a->ldw ? a->ldw : a->K, ldy = a->ldy ? a->ldy : a->N;
  if (ldx < a->K || ldw < a->K)
    return fail(SA_ERR_INVALID, "row strides of x and w must be >= K = %d (ldx=%lld ldw=%lld)", a->K, (long long)ldx,
                (long long)ldw);
  if (ldy < a->N) return fail(SA_ERR_INVALID, "row stride of y must be >= N = %d (ldy=%lld)", a->N, (long long)ldy);
  if (too_large(a->x_off) || too_large(a->y_off) || too_large(a->gate_off) || too_large(ldx) || too_large(ldw) ||
      too_large(ldy))
    return fail(SA_ERR_INVALID, "offsets and strides must be below 2^40 elements");
  if (!isfinite(a->alpha)) return fail(SA_ERR_INVALID, "alpha must be finite");
  if (a->act < SA_ACT_NONE || a->act > SA_ACT_SILU) return fail(SA_ERR_INVALID, "unknown act %d", a->act);
  if (a->epilogue < SA_EPI_STORE || a->epilogue > SA_EPI_RESID_GATE)
    return fail(SA_ERR_INVALID, "unknown epilogue %d", a->epilogue);
  if (a->epilogue == SA_EPI_RESID_GATE && !a->gate) return fail(SA_ERR_INVALID, "SA_EPI_RESID_GATE needs gate");
  // the output must not overlap what the kernel reads (it reads y itself only at the element it writes)
  const Extent ey = extent(a->y, a->y_off, 0, ldy, 1, a->M, a->N);
  const Extent ex = extent(a->x, a->x_off, 0, ldx, 1, a->M, a->K);
  const Extent ew = extent(a->w, 0, 0, ldw, 1, a->N, a->K);
  if (!ey.ok || !ex.ok || !ew.ok) return fail(SA_ERR_INVALID, "the extent of x, w or y overflows 64-bit addresses");
  if (overlaps(ey, ex) || overlaps(ey, ew)) return fail(SA_ERR_ALIAS, "y overlaps x or w");
  if (a->bias && overlaps(ey, extent(a->bias, 0, 0, 0, 1, 1, a->N))) return fail(SA_ERR_ALIAS, "y overlaps bias");
  if (a->epilogue == SA_EPI_RESID_GATE && overlaps(ey, extent(a->gate, a->gate_off, 0, 0, 1, 1, a->N)))
    return fail(SA_ERR_ALIAS, "y overlaps gate");
  p->x = a->x;
  p->x_off = a->x_off;
  p->ldx = ldx;
  p->w = a->w;
  p->ldw = ldw;
  p->bias = a->bias;
  p->gate = a->epilogue == SA_EPI_RESID_GATE ? a->gate : nullptr;
  p->gate_off = a->gate_off;
  p->y = a->y;
  p->y_off = a->y_off;
  p->ldy = ldy;
  p->resid = nullptr;
  p->M = a->M;
  p->N = a->N;
  p->K = a->K;
  p->alpha = a->alpha;
  p->act = a->act;
  p->epi = a->epilogue;
  if (!sa::linear_mfma_supported(*p) && (int64_t)a->M > (int64_t)65535 * 16)  // generic kernel grid
    return fail(SA_ERR_UNSUPPORTED, "M = %d exceeds the %d rows the unaligned / K %% 8 != 0 path supports", a->M,
                65535 * 16);
  return SA_OK;
}

// Workspace of the VAE block (byte offsets, 256-byte aligned parts): normalized image [HW, C],
// q|k|v [HW, 3C], attention output [HW, C], GroupNorm chunk statistics, then the attention call's
// own scratch.
struct VaeLayout {
  int64_t n, qkv, a, gn, attn, total;
};

int64_t align256(int64_t b) { return (b + 255) & ~(int64_t)255; }

// Sizes -> layout and the attention call over the q|k|v part of `ws` (any 256-byte aligned base
// gives the same kernel choice as the real workspace, which is 16-byte aligned at least).
int vae_plan(const sa_vae_attn_args* a, char* ws, VaeLayout* L, sa_attn_args* at);

enum class Path { kFlash, kSmall, kSmall16, kWide, kGeneric };

struct Choice {
  Path path;
  int nsplit;
  sa::WidePlan wide;
  const char* name;
};

// ---- per-device state: CU count (0 until queried; concurrent first calls query it twice, harmlessly)
constexpr int kMaxDevices = 64;
std::atomic<int> g_num_cus[kMaxDevices];

int current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return -1;
  return dev;
}

// CU count of the current device (256 on MI355X); the MI355X value when no device is visible, so
// that kernel selection can be inspected on a host without a GPU.
int num_cus() {
  const int dev = current_device();
  if (dev < 0) return 256;
  int n = g_num_cus[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
  g_num_cus[dev].store(n, std::memory_order_relaxed);
  return n;
}

// Kernel selection. The MFMA kernels need D in {64, 128} and 16-byte aligned rows (the same gate
// as the fused path of app/gpu/ops.js:111-112); everything else goes to the generic kernel.
int choose(const sa::AttnParams& p, Choice* c) {
  const bool vec = aligned16(p.q) && aligned16(p.k) && aligned16(p.v) && aligned16(p.o) && p.q_off % 4 == 0 &&
                   p.k_off % 4 == 0 && p.v_off % 4 == 0 && p.o_off % 4 == 0 && p.ldq % 4 == 0 && p.ldk % 4 == 0 &&
                   p.ldv % 4 == 0 && p.ldo % 4 == 0 && p.sq % 4 == 0 && p.sk % 4 == 0 && p.sv % 4 == 0 &&
                   p.so % 4 == 0;
  // The MFMA kernels address a copy's rows (up to 128) as 32-bit byte offsets from the block's
  // first row; longer strides take the generic kernel, whose addresses are 64-bit.
  const bool off32 = p.ldk < ((int64_t)1 << 22) && p.ldv < ((int64_t)1 << 22);
  if ((p.D == 64 || p.D == 128) && vec && off32 && sa::flash_mfma_args_fit(p)) {
    // Units of 32 queries. Head dim 64 with at most one unit per CU (the batch-2 DiT calls, a T5
    // prompt): one workgroup per unit with its key blocks dealt to 4 waves. Otherwise the
    // 128-query flash kernel, which below ~2 waves per SIMD (256 CUs x 4 SIMDs) splits the key
    // blocks across two waves of each workgroup.
    const int64_t units = (int64_t)p.B * p.H * ((p.Lq + 31) / 32);
    const int nblk = (p.Lk + 31) / 32;
    if (p.D == 64 && units <= sa::kSmallLaunchCUs && nblk >= 2) {
      // groups of 16 queries while they still fit one workgroup per CU (short sequences packed to
      // make them fit): twice the CUs, half the MFMA cycles per key block on each SIMD
      const bool g16 = sa::flash_small16_workgroups(p) <= sa::kSmallLaunchCUs;
      c->path = g16 ? Path::kSmall16 : Path::kSmall;
      c->nsplit = sa::flash_small_waves(p);
      c->name = g16 ? sa::flash_small16_name() : sa::flash_small_name(c->nsplit);
      return SA_OK;
    }
    int nsplit = 1;
    if (units < 2048 && nblk >= 2) nsplit = 2;
    c->path = Path::kFlash;
    c->nsplit = nsplit;
    c->name = sa::flash_mfma_name(p.D, nsplit);
    return SA_OK;
  }
  if (vec && off32 && sa::wide_mfma_supported(p)) {
    c->path = Path::kWide;
    c->nsplit = 1;
    c->wide = sa::wide_mfma_plan(p, num_cus());
    c->name = sa::wide_mfma_name(p.D);
    return SA_OK;
  }
  if (p.D > sa::GENERIC_MAX_D)
    return fail(SA_ERR_UNSUPPORTED, "head dim %d exceeds the supported maximum %d", p.D, sa::GENERIC_MAX_D);
  c->path = Path::kGeneric;
  c->nsplit = 1;
  c->name = "generic";
  return SA_OK;
}

// The sequence schedule of a key-length call whose host copy of the lengths came along: made for the
// chosen flash kernel (its units per sequence and workgroups per CU), and used only when the batch is
// large enough to queue workgroups (small batches run in one round) and the order is not the launch
// order already (the schedule pays one dependent kernel-argument load per workgroup).
void apply_schedule(sa::AttnParams& p, const Choice& c) {
  p.order_n = 0;
  if (c.path != Path::kFlash || p.key_len_host == nullptr || p.B < 8 || p.B > sa::kMaxOrder) return;
  ScheduleModel m;
  m.B = p.B;
  m.Lk = p.Lk;
  m.C = num_cus() / 8;
  m.S = sa::flash_mfma_per_cu(p, c.nsplit);
  const int qt = sa::flash_mfma_unit_queries(c.nsplit);
  m.T = (int64_t)p.H * ((p.Lq + qt - 1) / qt);
  cached_schedule(p.key_len_host, m, p.order);
  for (int r = 0; r < p.B; ++r)
    if (p.order[r] != r) {
      p.order_n = p.B;
      break;
    }
}

}  // namespace

namespace {

// ---- scratch of the allocation-free entry point: one static device array, which every GPU the
// library runs on holds (its own copy, at its own address) until the process ends. In host code
// `scratch` names a host-side stand-in, never the device memory: host code uses only the address
// hipGetSymbolAddress returns for the current device (kept per device in g_scratch).
constexpr int64_t kScratchBytes = SA_NOALLOC_SCRATCH_BYTES;
static_assert(kScratchBytes == sa::kWideMaxRecordBytes, "wide-head plans are sized to this scratch");
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
std::atomic<void*> g_scratch[kMaxDevices];

// Device address of the current device's scratch, looked up once per device: at the library's
// first use on that device (prepare_device), or failing that by the first allocation-free call.
int scratch_address(void** out) {
  const int dev = current_device();
  if (dev < 0) return fail(SA_ERR_HIP, "no current HIP device");
  void* ptr = g_scratch[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (ptr == nullptr) return fail(SA_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch[dev].store(ptr, std::memory_order_release);
  }
  *out = ptr;
  return SA_OK;
}

// Set-up of the current device at the library's first use there (sa_set_device, sa_malloc,
// sa_stream_create, any operator call): the scratch address lookup, which may load the library's
// device code on the device, so that an allocation-free call captured into a HIP graph later does
// neither. Errors are left to the allocation-free call, which looks up again and reports them.
void prepare_device() {
  const int dev = current_device();
  if (dev < 0 || g_scratch[dev].load(std::memory_order_acquire) != nullptr) return;
  char err[sizeof(g_err)];
  const int status = g_status;
  memcpy(err, g_err, sizeof err);
  void* ptr = nullptr;
  (void)scratch_address(&ptr);
  memcpy(g_err, err, sizeof err);  // the caller's own status stays as it was
  g_status = status;
}

// Validates, selects and launches one attention call. The wide-head kernel's merge records go to
// the caller's workspace, or (own_scratch) to the library's per-GPU scratch.
int run_attention(const sa_attn_args* args, void* stream, bool own_scratch) {
  prepare_device();
  sa::AttnParams p;
  int rc = resolve(args, &p);
  if (rc != SA_OK) return rc;
  Choice c;
  rc = choose(p, &c);
  if (rc != SA_OK) return rc;
  apply_schedule(p, c);
  hipError_t e;
  if (c.path == Path::kFlash) {
    e = sa::launch_flash_mfma(p, c.nsplit, num_cus(), (hipStream_t)stream);
  } else if (c.path == Path::kSmall) {
    e = sa::launch_flash_small(p, (hipStream_t)stream);
  } else if (c.path == Path::kSmall16) {
    e = sa::launch_flash_small16(p, (hipStream_t)stream);
  } else if (c.path == Path::kWide) {
    float* ws = nullptr;
    if (c.wide.ws_floats > 0) {
      const int64_t need = c.wide.ws_floats * (int64_t)sizeof(float);
      void* base = nullptr;
      if (own_scratch) {
        if (need > kScratchBytes)
          return fail(SA_ERR_UNSUPPORTED,
                      "this call needs %lld bytes of scratch, more than the %lld bytes sa_attention_f32_noalloc has "
                      "(pass a workspace to sa_attention_f32 instead)",
                      (long long)need, (long long)kScratchBytes);
        rc = scratch_address(&base);
        if (rc != SA_OK) return rc;
      } else {
        if (!args->workspace || args->workspace_bytes < need)
          return fail(SA_ERR_INVALID, "this call needs a device workspace of %lld bytes (sa_attention_workspace_bytes)",
                      (long long)need);
        if (!aligned16(args->workspace)) return fail(SA_ERR_INVALID, "workspace must be 16-byte aligned");
        base = args->workspace;
      }
      const Extent ew = {(uintptr_t)base, (uintptr_t)base + (uintptr_t)need, true};
      const int64_t HD = (int64_t)p.H * p.D;
      if (overlaps(ew, extent(p.o, p.o_off, p.so, p.ldo, p.B, p.Lq, HD)) ||
          overlaps(ew, extent(p.q, p.q_off, p.sq, p.ldq, p.B, p.Lq, HD)) ||
          overlaps(ew, extent(p.k, p.k_off, p.sk, p.ldk, p.B, p.Lk, HD)) ||
          overlaps(ew, extent(p.v, p.v_off, p.sv, p.ldv, p.B, p.Lk, HD)))
        return fail(SA_ERR_ALIAS, "the workspace overlaps q, k, v or o");
      ws = static_cast<float*>(base);
    }
    e = sa::launch_wide_mfma(p, c.wide, ws, (hipStream_t)stream);
  } else {
    e = sa::launch_generic(p, (hipStream_t)stream);
  }
  if (e != hipSuccess) return hip_fail(e, c.name);
  return ok();
}

}  // namespace

extern "C" {

int sa_attention_f32(const sa_attn_args* args, void* stream) { return run_attention(args, stream, false); }

int sa_attention_f32_noalloc(const sa_attn_args* args, void* stream) { return run_attention(args, stream, true); }

int64_t sa_attention_workspace_bytes(const sa_attn_args* args) {
  sa::AttnParams p;
  int rc = resolve(args, &p);
  if (rc != SA_OK) return rc;
  Choice c;
  rc = choose(p, &c);
  if (rc != SA_OK) return rc;
  ok();
  return c.path == Path::kWide ? c.wide.ws_floats * (int64_t)sizeof(float) : 0;
}

// The linear layer with an optional residual source (resid: rows laid out like y, read by the
// residual epilogues in place of y; the caller has checked that it does not overlap y).
static int run_linear(const sa_linear_args* args, const float* resid, void* stream) {
  prepare_device();
  sa::LinearParams p;
  const int rc = resolve_linear(args, &p);
  if (rc != SA_OK) return rc;
  p.resid = resid;
  const hipError_t e = sa::launch_linear(p, num_cus(), (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, sa::linear_kernel_name(p, num_cus()));
  return ok();
}

int sa_linear_f32(const sa_linear_args* args, void* stream) { return run_linear(args, nullptr, stream); }

const char* sa_linear_kernel_name(const sa_linear_args* args) {
  sa::LinearParams p;
  if (resolve_linear(args, &p) != SA_OK) return nullptr;
  ok();
  return sa::linear_kernel_name(p, num_cus());
}

int sa_vae_attention_f32(const sa_vae_attn_args* a, void* stream) {
  if (a == nullptr) return fail(SA_ERR_INVALID, "args is NULL");
  VaeLayout L;
  sa_attn_args at;
  int rc = vae_plan(a, static_cast<char*>(a->workspace), &L, &at);
  if (rc != SA_OK) return rc;
  if (!a->x || !a->gamma || !a->beta || !a->wqkv || !a->wo || !a->out)
    return fail(SA_ERR_INVALID, "x, gamma, beta, wqkv, wo and out must be non-NULL device pointers");
  if (!a->workspace || a->workspace_bytes < L.total)
    return fail(SA_ERR_INVALID, "this call needs a device workspace of %lld bytes (sa_vae_attention_workspace_bytes)",
                (long long)L.total);
  if (!aligned16(a->workspace)) return fail(SA_ERR_INVALID, "workspace must be 16-byte aligned");
  const int64_t HW = a->HW, C = a->C;
  auto span = [](const void* p, int64_t floats) -> Extent {
    return {(uintptr_t)p, (uintptr_t)p + (uintptr_t)(floats * 4), true};
  };
  const Extent ew = {(uintptr_t)a->workspace, (uintptr_t)a->workspace + (uintptr_t)L.total, true};
  const Extent ex = span(a->x, HW * C), eo = span(a->out, HW * C);
  if (overlaps(ew, ex) || overlaps(ew, eo)) return fail(SA_ERR_ALIAS, "the workspace overlaps x or out");
  if (a->out != a->x && overlaps(eo, ex)) return fail(SA_ERR_ALIAS, "out overlaps x (pass out == x to update in place)");
  const Extent params[] = {span(a->gamma, C), span(a->beta, C), span(a->wqkv, 3 * C * C),
                           span(a->bqkv, a->bqkv ? 3 * C : 0), span(a->wo, C * C), span(a->bo, a->bo ? C : 0)};
  for (const Extent& e : params)
    if (e.lo != e.hi && (overlaps(e, eo) || overlaps(e, ew)))
      return fail(SA_ERR_ALIAS, "out or the workspace overlaps a parameter");

  char* ws = static_cast<char*>(a->workspace);
  float* n = reinterpret_cast<float*>(ws + L.n);
  float* qkv = reinterpret_cast<float*>(ws + L.qkv);
  float* att = reinterpret_cast<float*>(ws + L.a);
  sa_linear_args l1 = {};
  l1.struct_size = sizeof l1;
  l1.M = a->HW;
  l1.N = 3 * a->C;
  l1.K = a->C;
  l1.x = n;
  l1.w = a->wqkv;
  l1.bias = a->bqkv;
  l1.alpha = 1.f;
  l1.y = qkv;
  sa_linear_args l2 = l1;
  l2.N = a->C;
  l2.x = att;
  l2.w = a->wo;
  l2.bias = a->bo;
  l2.epilogue = SA_EPI_RESID;
  l2.y = a->out;
  // every part is validated before the first launch, so a rejected call launches nothing
  if (!sa_linear_kernel_name(&l1) || !sa_attention_kernel_name(&at) || !sa_linear_kernel_name(&l2)) {
    // the rejecting part's own status (SA_ERR_UNSUPPORTED, SA_ERR_ALIAS, ...) and message
    const int why_rc = g_status != SA_OK ? g_status : SA_ERR_INVALID;
    char why[sizeof(g_err)];
    memcpy(why, g_err, sizeof why);
    return fail(why_rc, "VAE block: %s", why);
  }
  const hipStream_t st = (hipStream_t)stream;
  hipError_t e = sa::launch_groupnorm(a->x, a->gamma, a->beta, n, reinterpret_cast<float*>(ws + L.gn), a->HW, a->C,
                                      a->groups, a->eps, st);
  if (e != hipSuccess) return hip_fail(e, "groupnorm");
  if ((rc = sa_linear_f32(&l1, stream)) != SA_OK) return rc;
  if ((rc = sa_attention_f32(&at, stream)) != SA_OK) return rc;
  // out = x + a Wo^T + bo: the residual epilogue reads x directly when out is another buffer
  // (checked above not to overlap x)
  if ((rc = run_linear(&l2, a->out != a->x ? a->x : nullptr, stream)) != SA_OK) return rc;
  return ok();
}

int64_t sa_vae_attention_workspace_bytes(const sa_vae_attn_args* a) {
  VaeLayout L;
  sa_attn_args at;
  const int rc = vae_plan(a, reinterpret_cast<char*>((uintptr_t)1 << 40), &L, &at);
  if (rc != SA_OK) return rc;
  ok();
  return L.total;
}

const char* sa_attention_kernel_name(const sa_attn_args* args) {
  sa::AttnParams p;
  if (resolve(args, &p) != SA_OK) return nullptr;
  Choice c;
  if (choose(p, &c) != SA_OK) return nullptr;
  ok();
  return c.name;
}

int sa_attention_plan(const sa_attn_args* args, sa_attn_plan* plan) {
  if (plan == nullptr) return fail(SA_ERR_INVALID, "plan is NULL");
  const uint32_t size = plan->struct_size;
  if (!plan_size_ok(size))
    return fail(SA_ERR_INVALID, "plan struct_size %u does not match sizeof(sa_attn_plan) = %zu", size,
                sizeof(sa_attn_plan));
  sa::AttnParams p;
  int rc = resolve(args, &p);
  if (rc != SA_OK) return rc;
  Choice c;
  rc = choose(p, &c);
  if (rc != SA_OK) return rc;
  apply_schedule(p, c);  // as the launch would: the plan reports the order it would use
  // filled in full here, then copied out up to the caller's struct_size
  sa_attn_plan full{};
  sa_attn_plan* const out = plan;
  plan = &full;
  plan->struct_size = size;
  plan->name = c.name;
  plan->bias_mode = p.bias_mode;
  plan->mask_variant = p.mask_mode;
  if (c.path == Path::kFlash) {
    const sa::FlashVariant fv = sa::flash_mfma_variant(p, c.nsplit);
    plan->kernel = SA_KERNEL_FLASH;
    plan->head_dim = fv.D;
    plan->key_split = fv.nsplit;
    plan->mask_variant = fv.mask;
    plan->keys_per_step = 32 * fv.nsplit;
    plan->workgroups = sa::flash_mfma_workgroups(p, c.nsplit, num_cus());
    const int64_t tail = sa::flash_mfma_tail_units(p, c.nsplit, num_cus());
    if (tail > 0) {
      const int tk = sa::flash_mfma_tail_kernel(p, c.nsplit, num_cus());
      const bool small = tk == sa::TAIL_SMALL;
      plan->tail_kernel = small ? SA_KERNEL_FLASH_SMALL : SA_KERNEL_FLASH;
      plan->tail_key_split = small ? sa::flash_small_waves(p) : 2;
      int64_t first = 0;
      plan->tail_workgroups = sa::flash_mfma_tail_groups(p, c.nsplit, num_cus(), &first);
      plan->tail_folded = tk == sa::TAIL_FOLD ? 1 : 0;
    }
  } else if (c.path == Path::kSmall || c.path == Path::kSmall16) {
    const bool g16 = c.path == Path::kSmall16;
    plan->kernel = g16 ? SA_KERNEL_FLASH_SMALL16 : SA_KERNEL_FLASH_SMALL;
    plan->head_dim = p.D;
    plan->key_split = c.nsplit;
    plan->keys_per_step = 32 * c.nsplit;
    plan->workgroups = g16 ? sa::flash_small16_workgroups(p) : sa::flash_small_workgroups(p);
    if (g16) plan->mask_variant = sa::flash_small16_variant(p).mask;
  } else if (c.path == Path::kWide) {
    plan->kernel = SA_KERNEL_WIDE;
    plan->head_dim = p.D;
    const int64_t groups = (int64_t)p.B * p.H * c.wide.q_groups;
    if (c.wide.nks > 1 && c.wide.whole > 0) {  // whole rounds unsplit, then the rest in chunks
      plan->key_chunks = 1;
      plan->keys_per_step = c.wide.whole_chunk;
      plan->workgroups = c.wide.whole;
      plan->tail_kernel = SA_KERNEL_WIDE;
      plan->tail_key_split = c.wide.nks;
      plan->tail_workgroups = (groups - c.wide.whole) * c.wide.nks;
    } else {
      plan->key_chunks = c.wide.nks;
      plan->keys_per_step = c.wide.chunk;
      plan->workgroups = groups * c.wide.nks;
    }
    plan->workspace_bytes = c.wide.ws_floats * (int64_t)sizeof(float);
  } else {
    plan->kernel = SA_KERNEL_GENERIC;
    plan->head_dim = p.D;
    plan->workgroups = (int64_t)p.B * p.H * p.Lq;
  }
  if (plan->kernel == SA_KERNEL_FLASH && plan->mask_variant == SA_MASK_VARIANT_KEY_LEN_SCHEDULED) {
    plan->order_n = p.B;
    memcpy(plan->sequence_order, p.order, (size_t)p.B);
  }
  memcpy(out, plan, size);
  return ok();
}

int32_t sa_attention_variant_count(void) {
  // flash variants, small-launch variants (32-query, then 16-query groups), the wide kernels (D 256,
  // 512 x no bias / dense bias x no mask / key lengths / key mask), then generic
  return sa::flash_mfma_variants(nullptr, 0) + sa::flash_small_variants(nullptr, 0) +
         sa::flash_small16_variants(nullptr, 0) + sa::wide_mfma_variants(nullptr, 0) + 1;
}

int sa_attention_variant(int32_t index, sa_attn_plan* plan) {
  if (plan == nullptr) return fail(SA_ERR_INVALID, "plan is NULL");
  const uint32_t size = plan->struct_size;
  if (!plan_size_ok(size))
    return fail(SA_ERR_INVALID, "plan struct_size %u does not match sizeof(sa_attn_plan) = %zu", size,
                sizeof(sa_attn_plan));
  const int nflash = sa::flash_mfma_variants(nullptr, 0);
  const int nsmall = sa::flash_small_variants(nullptr, 0);
  const int nsmall16 = sa::flash_small16_variants(nullptr, 0);
  if (index < 0 || index >= sa_attention_variant_count())
    return fail(SA_ERR_INVALID, "variant index %d outside [0, %d)", index, sa_attention_variant_count());
  // filled in full here, then copied out up to the caller's struct_size
  sa_attn_plan full{};
  sa_attn_plan* const out = plan;
  plan = &full;
  plan->struct_size = size;
  if (index >= nflash && index < nflash + nsmall) {
    sa::FlashVariant v[64];
    if (sa::flash_small_variants(v, 64) > 64) return fail(SA_ERR_UNSUPPORTED, "variant table overflow");
    const sa::FlashVariant& x = v[index - nflash];
    plan->kernel = SA_KERNEL_FLASH_SMALL;
    plan->head_dim = x.D;
    plan->key_split = x.nsplit;
    plan->bias_mode = x.bias;
    plan->mask_variant = x.mask;
    plan->name = sa::flash_small_name(x.nsplit);
    memcpy(out, plan, size);
    return ok();
  }
  if (index >= nflash + nsmall && index < nflash + nsmall + nsmall16) {
    sa::FlashVariant v[64];
    if (sa::flash_small16_variants(v, 64) > 64) return fail(SA_ERR_UNSUPPORTED, "variant table overflow");
    const sa::FlashVariant& x = v[index - nflash - nsmall];
    plan->kernel = SA_KERNEL_FLASH_SMALL16;
    plan->head_dim = x.D;
    plan->key_split = x.nsplit;
    plan->bias_mode = x.bias;
    plan->mask_variant = x.mask;
    plan->name = sa::flash_small16_name();
    memcpy(out, plan, size);
    return ok();
  }
  if (index >= nflash) index -= nsmall + nsmall16;
  if (index < nflash) {
    sa::FlashVariant v[128];
    static_assert(sizeof(v) / sizeof(v[0]) >= 60, "variant table");
    const int n = sa::flash_mfma_variants(v, 128);
    if (n > 128) return fail(SA_ERR_UNSUPPORTED, "variant table overflow");
    plan->kernel = SA_KERNEL_FLASH;
    plan->head_dim = v[index].D;
    plan->key_split = v[index].nsplit;
    plan->bias_mode = v[index].bias;
    plan->mask_variant = v[index].mask;
    plan->name = sa::flash_mfma_name(v[index].D, v[index].nsplit);
  } else if (index < nflash + sa::wide_mfma_variants(nullptr, 0)) {
    sa::FlashVariant v[64];
    if (sa::wide_mfma_variants(v, 64) > 64) return fail(SA_ERR_UNSUPPORTED, "variant table overflow");
    const sa::FlashVariant& x = v[index - nflash];
    plan->kernel = SA_KERNEL_WIDE;
    plan->head_dim = x.D;
    plan->bias_mode = x.bias;
    plan->mask_variant = x.mask;
    plan->name = sa::wide_mfma_name(x.D);
  } else {
    plan->kernel = SA_KERNEL_GENERIC;
    plan->name = "generic";
  }
  memcpy(out, plan, size);
  return ok();
}

int sa_t5_bucket_lut(int32_t Lq, int32_t Lk, int32_t num_buckets, int32_t max_distance, int32_t bidirectional,
                     int32_t* out) {
  if (Lq < 1 || Lk < 1 || !out) return fail(SA_ERR_INVALID, "Lq, Lk must be >= 1 and out non-NULL");
  if (num_buckets < (bidirectional ? 4 : 2) || max_distance < 1)
    return fail(SA_ERR_INVALID, "num_buckets %d / max_distance %d out of range", num_buckets, max_distance);
  int nb = num_buckets;
  if (bidirectional) nb /= 2;
  const int max_exact = nb / 2;
  if (max_exact < 1 || max_distance <= max_exact)
    return fail(SA_ERR_INVALID, "max_distance must exceed num_buckets/%d", bidirectional ? 4 : 2);
  // float32 arithmetic as torch does it; log is rounded once from double (a correctly rounded
  // float32 log, like Math.fround(Math.log(x)) in app/models/t5.js:21).
  const float den = (float)log((double)max_distance / (double)max_exact);
  const int n_rel = Lq + Lk - 1;
  for (int idx = 0; idx < n_rel; ++idx) {
    const int rel = idx - (Lq - 1);
    int bucket = 0;
    int n;
    if (bidirectional) {
      if (rel > 0) bucket = nb;
      n = rel < 0 ? -rel : rel;
    } else {
      n = rel < 0 ? -rel : 0;
    }
    if (n < max_exact) {
      bucket += n;
    } else {
      const float ratio = (float)n / (float)max_exact;
      const float lg = (float)log((double)ratio);
      const float scaled = (lg / den) * (float)(nb - max_exact);
      int large = max_exact + (int)scaled;
      if (large > nb - 1) large = nb - 1;
      bucket += large;
    }
    out[idx] = bucket;
  }
  return ok();
}

int sa_t5_position_bias(const float* table, const int32_t* bucket_lut, int32_t num_buckets, int32_t H, int32_t Lq,
                        int32_t Lk, float* out, void* stream) {
  if (!table || !bucket_lut || !out) return fail(SA_ERR_INVALID, "table, bucket_lut and out must be non-NULL");
  if (num_buckets < 1 || H < 1 || Lq < 1 || Lk < 1) return fail(SA_ERR_INVALID, "sizes must be >= 1");
  hipError_t e = sa::launch_position_bias(table, bucket_lut, num_buckets, H, Lq, Lk, out, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "position_bias");
  return ok();
}

int sa_device_count(int32_t* count) {
  if (!count) return fail(SA_ERR_INVALID, "count is NULL");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) {
    *count = 0;
    return hip_fail(e, "hipGetDeviceCount");
  }
  *count = n;
  return ok();
}

int sa_set_device(int32_t device) {
  hipError_t e = hipSetDevice(device);
  if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
  prepare_device();
  return ok();
}

int sa_malloc(void** ptr, size_t bytes) {
  if (!ptr) return fail(SA_ERR_INVALID, "ptr is NULL");
  *ptr = nullptr;
  hipError_t e = hipMalloc(ptr, bytes == 0 ? 16 : bytes);
  if (e != hipSuccess) return hip_fail(e, "hipMalloc");
  prepare_device();
  return ok();
}

int sa_free(void* ptr) {
  if (!ptr) return ok();
  hipError_t e = hipFree(ptr);
  return e == hipSuccess ? ok() : hip_fail(e, "hipFree");
}

int sa_malloc_host(void** ptr, size_t bytes) {
  if (!ptr) return fail(SA_ERR_INVALID, "ptr is NULL");
  *ptr = nullptr;
  hipError_t e = hipHostMalloc(ptr, bytes == 0 ? 16 : bytes, hipHostMallocDefault);
  return e == hipSuccess ? ok() : hip_fail(e, "hipHostMalloc");
}

int sa_free_host(void* ptr) {
  if (!ptr) return ok();
  hipError_t e = hipHostFree(ptr);
  return e == hipSuccess ? ok() : hip_fail(e, "hipHostFree");
}

int sa_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
  if (bytes == 0) return ok();
  if (!dst || !src) return fail(SA_ERR_INVALID, "NULL pointer");
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream);
  if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);  // the host buffer may be reused at once
  return e == hipSuccess ? ok() : hip_fail(e, "memcpy h2d");
}

int sa_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
  if (bytes == 0) return ok();
  if (!dst || !src) return fail(SA_ERR_INVALID, "NULL pointer");
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream);
  if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(e, "memcpy d2h");
}

int sa_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
  if (bytes == 0) return ok();
  if (!dst || !src) return fail(SA_ERR_INVALID, "NULL pointer");
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(e, "memcpy d2d");
}

int sa_memset(void* dst, int value, size_t bytes, void* stream) {
  if (bytes == 0) return ok();
  if (!dst) return fail(SA_ERR_INVALID, "NULL pointer");
  hipError_t e = hipMemsetAsync(dst, value, bytes, (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(e, "hipMemsetAsync");
}

int sa_stream_create(void** stream) {
  if (!stream) return fail(SA_ERR_INVALID, "stream is NULL");
  hipStream_t s = nullptr;
  hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  *stream = s;
  if (e != hipSuccess) return hip_fail(e, "hipStreamCreateWithFlags");
  prepare_device();
  return ok();
}

int sa_stream_destroy(void* stream) {
  if (!stream) return ok();
  hipError_t e = hipStreamDestroy((hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(e, "hipStreamDestroy");
}

int sa_stream_sync(void* stream) {
  hipError_t e = hipStreamSynchronize((hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(e, "hipStreamSynchronize");
}

int sa_device_sync(void) {
  hipError_t e = hipDeviceSynchronize();
  return e == hipSuccess ? ok() : hip_fail(e, "hipDeviceSynchronize");
}

int sa_event_create(void** event) {
  if (!event) return fail(SA_ERR_INVALID, "event is NULL");
  hipEvent_t ev = nullptr;
  hipError_t e = hipEventCreate(&ev);
  *event = ev;
  return e == hipSuccess ? ok() : hip_fail(e, "hipEventCreate");
}

int sa_event_destroy(void* event) {
  if (!event) return ok();
  hipError_t e = hipEventDestroy((hipEvent_t)event);
  return e == hipSuccess ? ok() : hip_fail(e, "hipEventDestroy");
}

int sa_event_record(void* event, void* stream) {
  if (!event) return fail(SA_ERR_INVALID, "event is NULL");
  hipError_t e = hipEventRecord((hipEvent_t)event, (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(e, "hipEventRecord");
}

int sa_event_elapsed_ms(float* ms, void* start, void* stop) {
  if (!ms || !start || !stop) return fail(SA_ERR_INVALID, "NULL pointer");
  hipError_t e = hipEventSynchronize((hipEvent_t)stop);
  if (e == hipSuccess) e = hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop);
  return e == hipSuccess ? ok() : hip_fail(e, "hipEventElapsedTime");
}

int sa_version(void) { return SA_ABI_VERSION; }

const char* sa_last_error(void) { return g_err; }

int sa_last_status(void) { return g_status; }

}  // extern "C"

namespace {

int vae_plan(const sa_vae_attn_args* a, char* ws, VaeLayout* L, sa_attn_args* at) {
  if (a == nullptr) return fail(SA_ERR_INVALID, "args is NULL");
  if (a->struct_size != sizeof(sa_vae_attn_args))
    return fail(SA_ERR_INVALID, "struct_size %u does not match sizeof(sa_vae_attn_args) = %zu", a->struct_size,
                sizeof(sa_vae_attn_args));
  if (a->HW <= 0 || a->C <= 0 || a->groups <= 0)
    return fail(SA_ERR_INVALID, "HW, C and groups must be positive (got %d, %d, %d)", a->HW, a->C, a->groups);
  if (a->C % a->groups != 0) return fail(SA_ERR_INVALID, "C = %d is not a multiple of groups = %d", a->C, a->groups);
  if (a->groups > 8192) return fail(SA_ERR_UNSUPPORTED, "at most 8192 GroupNorm groups");
  if (!(a->eps >= 0.f) || !isfinite(a->eps)) return fail(SA_ERR_INVALID, "eps must be finite and >= 0");
  if ((int64_t)a->C * 3 > 0x7fffffff) return fail(SA_ERR_UNSUPPORTED, "C too large");
  if (ws == nullptr) ws = reinterpret_cast<char*>((uintptr_t)1 << 40);  // layout only; checked by the caller
  const int64_t HW = a->HW, C = a->C;
  L->n = 0;
  L->qkv = align256(HW * C * 4);
  L->a = L->qkv + align256(HW * 3 * C * 4);
  L->gn = L->a + align256(HW * C * 4);
  L->attn = L->gn + align256((int64_t)3 * a->groups * sa::groupnorm_chunks(a->HW, a->groups) * 4);
  *at = sa_attn_args{};
  at->struct_size = sizeof(sa_attn_args);
  at->B = 1;
  at->H = 1;
  at->D = a->C;
  at->Lq = a->HW;
  at->Lk = a->HW;
  float* qkv = reinterpret_cast<float*>(ws + L->qkv);
  at->q = at->k = at->v = qkv;
  at->k_off = C;
  at->v_off = 2 * C;
  at->ldq = at->ldk = at->ldv = 3 * C;
  at->o = reinterpret_cast<float*>(ws + L->a);
  at->ldo = C;
  at->scale = 1.f / sqrtf((float)a->C);  // diffusers Attention default scale (vae.js:86: ops.js default)
  const int64_t attn_bytes = sa_attention_workspace_bytes(at);
  if (attn_bytes < 0) return (int)attn_bytes;
  at->workspace = attn_bytes > 0 ? ws + L->attn : nullptr;
  at->workspace_bytes = attn_bytes;
  L->total = L->attn + align256(attn_bytes);
  return SA_OK;
}

}  // namespace
