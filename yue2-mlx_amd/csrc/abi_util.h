// Host-side error and string helpers shared by the C ABI translation units.
// Errors follow the reference's types.hpp:21-25 convention (a type string
// and a message); no exception crosses the ABI (bridge.mm:147-157): guarded()
// maps them to status codes 0/1/2/130 (lyra.h:18-23) and an error JSON owned
// by the caller.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>

#include "../../include/yuear.h"

namespace yuear {
namespace {

struct Error : std::runtime_error {
  std::string type;
  Error(std::string t, const std::string &m) : std::runtime_error(m), type(std::move(t)) {}
};
[[noreturn]] void invalid(const std::string &m) { throw Error("ValueError", m); }

void hip_check(hipError_t e, const char *what) {
  if (e != hipSuccess)
    throw Error("RuntimeError", std::string(what) + ": " + hipGetErrorString(e));
}
#define HIPC(x) hip_check((x), #x)

std::string json_escape(const std::string &s) {
  std::string o;
  for (char c : s) {
    switch (c) {
    case '"': o += "\\\""; break;
    case '\\': o += "\\\\"; break;
    case '\n': o += "\\n"; break;
    default:
      if (static_cast<unsigned char>(c) < 0x20) {
        char buf[8];
        std::snprintf(buf, sizeof buf, "\\u%04x", c);
        o += buf;
      } else {
        o += c;
      }
    }
  }
  return o;
}
char *dup_string(const std::string &s) {
  char *p = static_cast<char *>(std::malloc(s.size() + 1));
  if (p)
    std::memcpy(p, s.c_str(), s.size() + 1);
  return p;
}
yuear_status fail(char **error_json, const std::string &type, const std::string &msg,
                  yuear_status st) {
  if (error_json)
    *error_json = dup_string("{\"type\":\"" + json_escape(type) + "\",\"message\":\"" +
                             json_escape(msg) + "\"}");
  return st;
}
template <class F> yuear_status guarded(char **error_json, F &&f) {
  if (error_json)
    *error_json = nullptr;
  try {
    f();
    return YUEAR_SUCCESS;
  } catch (const Error &e) {
    const yuear_status st = e.type == "InterruptedError" ? YUEAR_CANCELLED
                            : e.type == "ValueError"     ? YUEAR_INVALID_INPUT
                                                         : YUEAR_FAILURE;
    return fail(error_json, e.type, e.what(), st);
  } catch (const std::exception &e) {
    return fail(error_json, "RuntimeError", e.what(), YUEAR_FAILURE);
  } catch (...) {
    return fail(error_json, "RuntimeError", "unknown error", YUEAR_FAILURE);
  }
}

}  // namespace
}  // namespace yuear
