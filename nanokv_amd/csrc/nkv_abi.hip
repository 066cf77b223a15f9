// nkv_abi.hip -- library-wide C ABI entry points: version and error text.
#include "nkv_common.h"

namespace nkv {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

}  // namespace nkv

extern "C" int nkv_abi_version(void) { return NKV_ABI_VERSION; }

extern "C" const char* nkv_last_error(void) { return nkv::g_last_error.c_str(); }
