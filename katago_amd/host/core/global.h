// Minimal stand-in for KataGo's cpp/core/global.h: only what the neural-net
// backend boundary uses (StringError, a few string helpers, unique_ptr_void).
// Names and meanings follow /root/reference/cpp/core/global.h:35-262 so that a
// backend written against this header compiles unchanged against KataGo's.
#ifndef KATAGO_AMD_CORE_GLOBAL_H
#define KATAGO_AMD_CORE_GLOBAL_H

#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

class StringError : public std::exception {
 public:
  explicit StringError(const char* m) : message(m) {}
  explicit StringError(const std::string& m) : message(m) {}
  const char* what() const noexcept override { return message.c_str(); }
 private:
  std::string message;
};

namespace Global {
  std::string intToString(int x);
  std::string int64ToString(int64_t x);
  std::string floatToString(float x);
  std::string doubleToString(double x);
  bool isSuffix(const std::string& s, const std::string& suffix);
  std::string toLower(const std::string& s);
  std::string strprintf(const char* fmt, ...);
  [[noreturn]] void fatalError(const std::string& s);
}

#define ASSERT_UNREACHABLE (Global::fatalError(std::string("unreachable: ") + __FILE__ + " " + Global::intToString(__LINE__)))

// Type-erased owning pointer used by the block lists of the model descriptors
// (same shape as KataGo's core/global.h:254-262).
using unique_ptr_void = std::unique_ptr<void, void(*)(const void*)>;
template<typename T>
unique_ptr_void make_unique_void(T* ptr) {
  return unique_ptr_void(ptr, [](const void* p) { delete static_cast<const T*>(p); });
}

#endif
