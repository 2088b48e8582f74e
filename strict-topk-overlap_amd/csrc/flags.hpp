// Flag slots of the one-launch kernels (k_step1, k_spec1).
//
// A one-launch kernel hands data from producer workgroups to consumer
// workgroups of the same grid through flags: a producer stores its data,
// waits until the stores have completed, then sets a flag; a consumer polls
// the flag (bounded in time) and then reads the data, both with
// agent-coherent accesses.  The flags must be zero before a launch, and
// every launch leaves them zero (each consumer clears what it consumed).
// They live in static device memory inside the library (step.hip), in
// slots of kFlagSlotWords words: each stream takes a slot of its own on
// first use, so launches in flight on different streams never share flags,
// and launches on one stream are ordered.  The last word of a slot counts
// timed-out waits.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace stk {

constexpr size_t kFlagSlotWords = 16384;

// The flag slot of `stream` (*flags = nullptr when every slot is taken or
// `words` do not fit beside the time-out counter at flags[kFlagSlotWords -
// 1]).  The slots' device address is looked up on a device's first call;
// under stream capture that lookup is refused: an error, or with `quiet` a
// null slot (the caller runs its multi-launch form instead).
int flag_slot(hipStream_t stream, size_t words, bool quiet, uint32_t** flags);

// The longest wait of a one-launch kernel, in ticks of the 100 MHz counter.
uint64_t flag_spin();
// Failure tests only: the producers publish no flag (every wait times out).
int flag_drop();
// False when a test has asked for the multi-launch forms only.
bool flag_one_launch();

}  // namespace stk
