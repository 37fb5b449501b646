// Stand-in for KataGo's cpp/core/commontypes.h (enabled_t tri-state flag).
#ifndef KATAGO_AMD_CORE_COMMONTYPES_H
#define KATAGO_AMD_CORE_COMMONTYPES_H
#include <string>

struct enabled_t {
  enum value { False, True, Auto };
  value x;
  enabled_t() = default;
  constexpr enabled_t(value a) : x(a) {}
  explicit operator bool() = delete;
  constexpr bool operator==(enabled_t a) const { return x == a.x; }
  constexpr bool operator!=(enabled_t a) const { return x != a.x; }
  std::string toString() const { return x == True ? "true" : x == False ? "false" : "auto"; }
};
#endif
