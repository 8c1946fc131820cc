// Library-wide C entry points: version string and per-thread error message.
#include <cstring>
#include <string>

#include <hip/hip_runtime.h>

#include "zmoe_host.h"

namespace zmoe {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

}  // namespace zmoe

#ifndef ZMOE_SOURCE_HASH
#define ZMOE_SOURCE_HASH "unknown"
#endif

// "zmlx_amd <version> gfx950 src:<hash>", the hash of the sources the library
// was built from (zmlx_amd/build.py source_hash()).
extern "C" const char* zmoe_version(void) { return "zmlx_amd 0.1.0 gfx950 src:" ZMOE_SOURCE_HASH; }

extern "C" const char* zmoe_last_error(void) { return zmoe::g_last_error.c_str(); }

extern "C" unsigned* zmoe_host_flags_alloc(int n) {
  if (n <= 0) return nullptr;
  void* p = nullptr;
  if (hipHostMalloc(&p, static_cast<size_t>(n) * sizeof(unsigned), hipHostMallocMapped | hipHostMallocCoherent) !=
      hipSuccess)
    return nullptr;
  std::memset(p, 0, static_cast<size_t>(n) * sizeof(unsigned));
  return static_cast<unsigned*>(p);
}

extern "C" void zmoe_host_flags_free(unsigned* flags) {
  if (flags) (void)hipHostFree(flags);
}
