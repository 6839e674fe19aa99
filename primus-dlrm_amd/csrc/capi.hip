// Library-wide C ABI entry points: version and thread-local error text.
#include <cstring>
#include <string>

#include "pdm_common.h"

namespace pdm {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

}  // namespace pdm

extern "C" int32_t pdm_abi_version(void) { return 10000; }

extern "C" size_t pdm_last_error(char* buf, size_t n) {
  const std::string& e = pdm::g_last_error;
  if (buf && n > 0) {
    const size_t k = e.size() < n - 1 ? e.size() : n - 1;
    std::memcpy(buf, e.data(), k);
    buf[k] = '\0';
  }
  return e.size();
}
