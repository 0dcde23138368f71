// Grid-wide hand-off probe: the mechanisms a persistent kernel can use to pass a vector between
// all of its workgroups, timed alone (measurement hook; no reference counterpart). 256
// workgroups of 256 threads, one per CU, run `n_phases` phases; in every phase each workgroup
// publishes its slice of an n-word vector and waits until it has seen every other workgroup's.
//
//   IRON_HANDOFF_TAGGED   the persistent decode kernel's own mechanism, run by its own helpers
//                         (decode_persistent.hip: put_word_copies, gather_words): 64-bit
//                         {tag, payload} words in 8 copies, polled from the XCD's copy;
//   IRON_HANDOFF_COUNTER  one atomic counter for the grid, polled until every workgroup has
//                         arrived (a grid barrier; the vector is not exchanged);
//   IRON_HANDOFF_FLAGS    the slice is written with plain stores, then one device-scope fence
//                         (L2 write-back) and a per-workgroup flag; consumers poll all flags,
//                         fence once (L2 invalidate) and read the vector with plain loads;
//   IRON_HANDOFF_XCD_L2   the decode kernel's XCD-local hand-off (decode_persistent.hip): the
//                         32 workgroups of each XCD exchange their own n-word vector through the
//                         XCD's L2 (sc0 stores, nt polls);
//   IRON_HANDOFF_XCD_AGENT the same groups with device-scope words, for comparison.
//
// Every wait is bounded; a workgroup whose wait fails raises the error word and stops, and the
// others then fail their own waits, so the grid always drains.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"
#include "internal.h"

namespace {

constexpr int kProbeWGs = 256;
constexpr int kProbeMaxWords = iron::kHandoffMaxWords;
constexpr long long kProbeSpin = 1ll << 20;

struct ProbeParams {
  unsigned long long* vec;  // [2][n] words (flag mode)
  unsigned int* ctr;        // [1] arrival counter (counter mode)
  unsigned int* flags;      // [kProbeWGs] phase flags (flag mode)
  unsigned int* err;        // [1] error flag
  int n, n_phases;
  unsigned int base;        // tags and flags of this launch: base + phase + 1
};

// True in every thread if `v` is set in any thread of the workgroup.
IRON_DEV bool any_of(bool v) { return __syncthreads_or(v) != 0; }

template <int MODE>
__global__ __launch_bounds__(256) void handoff_probe_kernel(ProbeParams p) {
  const int wg = blockIdx.x, t = threadIdx.x, per = p.n / kProbeWGs;
  float acc = 0.f;
  for (int ph = 0; ph < p.n_phases; ++ph) {
    const unsigned int tag = p.base + (unsigned int)ph + 1u;
    unsigned long long* buf = p.vec + (size_t)(ph & 1) * p.n;
    bool failed = false;
    if constexpr (MODE == IRON_HANDOFF_COUNTER) {
      __syncthreads();
      if (t == 0) {
        __hip_atomic_fetch_add(p.ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const unsigned int want = (unsigned int)(kProbeWGs * (ph + 1));
        for (long long s = 0;; ++s) {
          if (__hip_atomic_load(p.ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= want)
            break;
          if (s >= kProbeSpin ||
              __hip_atomic_load(p.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
            failed = true;
            break;
          }
        }
      }
    } else {
      // plain stores; one device-scope fence (L2 write-back) and the flag from thread 0; the
      // consumers' flag polls; one fence (L2 invalidate) from thread 0; plain loads
      if (t < per)
        buf[(size_t)wg * per + t] = ((unsigned long long)tag << 32) | (unsigned int)(ph + wg);
      __syncthreads();
      if (t == 0) {
        __threadfence();
        __hip_atomic_store(p.flags + wg, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      for (long long s = 0;; ++s) {  // thread t watches workgroup t's flag
        // any tag at or past this phase's: a fast workgroup may already have raised its flag
        // for the next phase before this watcher saw this phase's value
        const unsigned int f =
            __hip_atomic_load(p.flags + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if ((int)(f - tag) >= 0) break;
        if (s >= kProbeSpin ||
            __hip_atomic_load(p.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
          failed = true;
          break;
        }
      }
      __syncthreads();
      if (t == 0) __threadfence();
      __syncthreads();
      for (int i = t; i < p.n; i += 256) acc += (float)(unsigned int)buf[i];
    }
    if (any_of(failed)) {
      if (t == 0) atomicOr(p.err, 1u);
      break;
    }
  }
  if (acc == -1.f) p.err[1] = 1u;  // keeps the consumed words live; never true
}

}  // namespace

extern "C" {

// Layout: the vector words (the tagged mode's replicated buffers, which also hold the flag mode's
// [2][n] vector), then 4 KiB: the counter at +0, the error word at +256, the flags at +1024.
static size_t probe_vec_bytes() { return iron::handoff_tagged_bytes(); }

// n_words: a multiple of 256 (a multiple of 32 is enough for the XCD modes), at most 2048.
size_t iron_handoff_probe_workspace(int n_words) {
  if (n_words <= 0 || n_words > kProbeMaxWords || n_words % (kProbeWGs / 8)) return 0;
  return probe_vec_bytes() + 4096;
}

int iron_handoff_probe(int mode, int n_words, int n_phases, unsigned int base, void* workspace,
                       size_t workspace_bytes, void* stream) {
  iron::clear_error();
  const char* fn = "iron_handoff_probe";
  if (mode != IRON_HANDOFF_TAGGED && mode != IRON_HANDOFF_COUNTER && mode != IRON_HANDOFF_FLAGS &&
      mode != IRON_HANDOFF_XCD_L2 && mode != IRON_HANDOFF_XCD_AGENT)
    return iron::fail(IRON_ERR_SHAPE, "%s: unknown mode %d", fn, mode);
  const bool xcd = mode == IRON_HANDOFF_XCD_L2 || mode == IRON_HANDOFF_XCD_AGENT;
  const int unit = xcd ? kProbeWGs / 8 : kProbeWGs;  // every workgroup publishes whole words
  if (n_words <= 0 || n_words > kProbeMaxWords || n_words % unit || n_phases <= 0)
    return iron::fail(IRON_ERR_SHAPE, "%s: n_words %d (a multiple of %d up to %d), phases %d", fn,
                      n_words, unit, kProbeMaxWords, n_phases);
  const size_t need = iron_handoff_probe_workspace(n_words);
  if (!workspace || workspace_bytes < need)
    return iron::fail(IRON_ERR_WORKSPACE, "%s: workspace %zu < %zu bytes", fn, workspace_bytes,
                      need);
  if (!iron::aligned(workspace, 256))
    return iron::fail(IRON_ERR_ALIGN, "%s: workspace not 256-byte aligned", fn);
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return iron::fail(IRON_ERR_HIP, "%s: device query failed", fn);
  if (cus < kProbeWGs)
    return iron::fail(IRON_ERR_UNSUPPORTED, "%s: needs %d CUs to hold the grid, device has %d",
                      fn, kProbeWGs, cus);
  ProbeParams p;
  char* b = (char*)workspace;
  p.vec = (unsigned long long*)b;
  char* tail = b + probe_vec_bytes();
  p.ctr = (unsigned int*)tail;
  p.err = (unsigned int*)(tail + 256);
  p.flags = (unsigned int*)(tail + 1024);
  p.n = n_words;
  p.n_phases = n_phases;
  p.base = base;
  hipStream_t s = (hipStream_t)stream;
  if (mode == IRON_HANDOFF_TAGGED)
    return iron::handoff_tagged_launch(workspace, p.err, n_words, n_phases, base, s);
  if (mode == IRON_HANDOFF_XCD_L2 || mode == IRON_HANDOFF_XCD_AGENT)
    return iron::handoff_xcd_launch(mode == IRON_HANDOFF_XCD_L2, workspace, p.err, n_words,
                                    n_phases, base, s);
  if (mode == IRON_HANDOFF_COUNTER)
    hipLaunchKernelGGL(handoff_probe_kernel<IRON_HANDOFF_COUNTER>, dim3(kProbeWGs), dim3(256), 0,
                       s, p);
  else
    hipLaunchKernelGGL(handoff_probe_kernel<IRON_HANDOFF_FLAGS>, dim3(kProbeWGs), dim3(256), 0, s,
                       p);
  return iron::check_launch(fn);
}

}  // extern "C"
