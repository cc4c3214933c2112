// Shared host-side helpers: status codes, the thread-local error text, and
// the exception type used inside the library (never crosses the C ABI).
#ifndef RAI_COMMON_H
#define RAI_COMMON_H

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "rai_hip.h"

namespace rai {

struct Error : std::runtime_error {
  rai_status code;
  Error(rai_status c, const std::string &m) : std::runtime_error(m), code(c) {}
};

[[noreturn]] inline void fail(rai_status c, const std::string &m) { throw Error(c, m); }

void set_last_error(const std::string &m);

inline size_t ceil_div(size_t a, size_t b) { return (a + b - 1) / b; }

inline size_t checked_mul(size_t a, size_t b, const char *what) {
  if (a != 0 && b > SIZE_MAX / a) fail(RAI_E_FORMAT, std::string(what) + " overflows");
  return a * b;
}
inline size_t checked_add(size_t a, size_t b, const char *what) {
  if (b > SIZE_MAX - a) fail(RAI_E_FORMAT, std::string(what) + " overflows");
  return a + b;
}

}  // namespace rai

// Wrap a C-ABI body: library exceptions become status codes + last error.
#define RAI_API_BODY(...)                                      \
  try {                                                        \
    __VA_ARGS__;                                               \
    return RAI_OK;                                             \
  } catch (const rai::Error &e) {                              \
    rai::set_last_error(e.what());                             \
    return e.code;                                             \
  } catch (const std::bad_alloc &) {                           \
    rai::set_last_error("host allocation failed");             \
    return RAI_E_OOM;                                          \
  } catch (const std::exception &e) {                          \
    rai::set_last_error(e.what());                             \
    return RAI_E_ARG;                                          \
  }

#endif
