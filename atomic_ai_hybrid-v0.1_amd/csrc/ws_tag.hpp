// Host-side record of which forward a caller's workspace holds, so that a
// backward asked to reuse the forward's intermediates (the *_REUSE flags) can
// refuse a workspace that does not hold the matching forward: never written
// by a saving forward, written for other inputs or shapes, or overwritten
// since by another call of this library.  Keyed by the workspace's address
// range; the inputs are compared by address (a caller that rewrites an input
// tensor in place between the two calls is not detected).
#pragma once
#include <cstddef>
#include <cstdint>

namespace ah {

struct WsTag {
  int kind;              // which forward wrote the workspace
  int32_t dims[8];       // its shape / dtype arguments
  const void* ptrs[8];   // its input pointers
  int64_t strides[8];    // its inputs' row strides (0 where dense)
};

// Forget every record overlapping [ws, ws + bytes): the caller's call writes there.
void ws_tag_clobber(const void* ws, size_t bytes);
// Forget overlapping records, then record that [ws, ws + bytes) holds t's forward.
void ws_tag_set(const void* ws, size_t bytes, const WsTag& t);
// Whether the workspace at ws was last recorded as holding t's forward.
bool ws_tag_matches(const void* ws, const WsTag& t);

}  // namespace ah
