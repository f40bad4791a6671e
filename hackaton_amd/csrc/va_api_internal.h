// Error reporting shared by the C-ABI translation units.
#pragma once

#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "../../include/varlen_attn.h"

namespace va {

// Thread-local message of the last failure (returned by va_last_error).
char* last_error_buffer();

// Formats the message into the thread's buffer and returns `code`.
inline int fail(int code, const char* fmt, ...) {
  char* buf = last_error_buffer();
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, 512, fmt, ap);
  va_end(ap);
  return code;
}

// va_bwd / va_bwd_stage / va_bwd_rotary_stage after argument validation (stage -1: both stages;
// rope NULL: no rotary epilogue). Shared with the entry point that brings its own scratch memory
// instead of a workspace argument.
int bwd_checked(int32_t stage, const void* dout, const void* q, const void* k, const void* v,
                const void* out, const float* lse, const int32_t* items, int64_t n_items,
                int64_t total_tokens, int32_t hq, int32_t hkv, int32_t head_dim, float scale,
                int32_t dtype, void* dq, void* dk, void* dv, void* workspace,
                int64_t workspace_bytes, void* stream, const va_rope_tables* rope);

}  // namespace va
