// nkv_internal.h -- entry points shared between the translation units of
// libnanokv_hip.so (not part of the C ABI).
#pragma once

#include "nkv_common.h"

namespace nkv {

// Key-chunk schedule of nkv_attend (nkv_chunk.hip).
int chunk_check(const nkv_attend_args* a);
size_t chunk_workspace_bytes(const nkv_attend_args* a);
int chunk_attend_launch(hipStream_t s, const nkv_attend_args* a, void* workspace,
                        size_t workspace_bytes);

}  // namespace nkv
