// kq_chain.h -- the resident decode chain (kq_chain.hip): host interface.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace kq {

// One step: y[out_dim] = W x for packed W of `kind`.  x is 16-byte aligned.
struct ChainStepDesc {
  int kind, in_dim, out_dim;
  const void* packed;
  const float* x;
  float* y;
};

struct Chain;

// Validates the steps (a step's x either lies inside exactly the latest
// earlier step's y that it overlaps -- its producer -- or is an input of the
// launch; no step writes memory an earlier step reads or writes) and
// allocates the chain's flags, counters and partial sums.  `why` names the
// violated rule on failure.
hipError_t chain_create(const ChainStepDesc* steps, int n, Chain** out, const char** why);
// One launch running every step; allocates nothing.  Launches of one chain
// must be ordered (one stream).
hipError_t chain_run(Chain* c, hipStream_t s);
// Synchronous: whether a dependency wait gave up since the last check (its
// rows may then be wrong), and clears the record.
hipError_t chain_check(Chain* c, unsigned* failed);
void chain_destroy(Chain* c);
int chain_workgroups(const Chain* c);

}  // namespace kq
