// Host-side helpers shared by the runtime's translation units (not part of the C ABI).
#pragma once

#include <stdint.h>

#include "../../include/strata_moe.h"

extern "C" {
// Resolves a view of a buffer registered with `ctx` to a device address after the ownership,
// extent (`need` bytes) and alignment checks of the coordinators: SM_E_OWNERSHIP or SM_E_VIEW
// on failure.
sm_status sm_internal_resolve_view(sm_context* ctx, sm_view v, uint64_t need, uint64_t align, uintptr_t* out);
// Makes the context's device current for the calling thread (SM_E_DEVICE if it cannot).
sm_status sm_internal_make_current(sm_context* ctx);
// Reads `bytes` of the GGUF file at absolute offset `offset` into host memory (SM_E_FILE if the
// file is shorter).
sm_status sm_internal_gguf_read(const sm_gguf* gguf, uint64_t offset, uint64_t bytes, void* dst);
}
