// Host-side helpers shared by the library's sources: the per-thread error
// message behind skv_last_error(), launch checking, dtype sizes, alignment,
// and the raw buffer descriptor constants used by the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "speech_kv.h"

namespace skv {

// Records a printf-style message for skv_last_error() and returns code.
int fail(int code, const char* fmt, ...);
// SKV_OK, or the pending launch error (recorded with `what`).
int check_launch(const char* what);
// Bytes per element of a dtype code; 0 if unknown.
int elt_bytes(int32_t dtype);

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Raw buffer descriptors (gfx9 word 3: 32-bit dword format) and the load
// cache hint for data read once (nontemporal).
constexpr int kBufWord3 = 0x00020000;
constexpr int kBufNt = 2;
// Byte offset past any descriptor range used here: such a load returns zeros.
constexpr uint32_t kBufOutOfRange = 0x80000000u;

}  // namespace skv
