#include "global.h"

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <iostream>

std::string Global::intToString(int x) { return std::to_string(x); }
std::string Global::int64ToString(int64_t x) { return std::to_string(x); }
std::string Global::floatToString(float x) { char buf[64]; snprintf(buf, sizeof(buf), "%g", (double)x); return buf; }
std::string Global::doubleToString(double x) { char buf[64]; snprintf(buf, sizeof(buf), "%g", x); return buf; }
bool Global::isSuffix(const std::string& s, const std::string& suffix) {
  return s.size() >= suffix.size() && s.compare(s.size() - suffix.size(), suffix.size(), suffix) == 0;
}
std::string Global::toLower(const std::string& s) {
  std::string r = s;
  for(char& c : r) if(c >= 'A' && c <= 'Z') c = (char)(c - 'A' + 'a');
  return r;
}
std::string Global::strprintf(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  va_list ap2;
  va_copy(ap2, ap);
  int n = vsnprintf(nullptr, 0, fmt, ap);
  va_end(ap);
  std::string out(n > 0 ? (size_t)n : 0, '\0');
  if(n > 0) vsnprintf(&out[0], (size_t)n + 1, fmt, ap2);
  va_end(ap2);
  return out;
}
void Global::fatalError(const std::string& s) {
  std::cerr << "FATAL: " << s << std::endl;
  std::abort();
}
