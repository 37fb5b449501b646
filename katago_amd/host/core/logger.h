// Stand-in for KataGo's cpp/core/logger.h: a Logger that backends may write
// informational lines to. Only write() is part of the backend-facing surface.
#ifndef KATAGO_AMD_CORE_LOGGER_H
#define KATAGO_AMD_CORE_LOGGER_H
#include <iostream>
#include <mutex>
#include <string>

class Logger {
 public:
  explicit Logger(std::ostream* out = &std::cerr) : out_(out) {}
  void write(const std::string& str) {
    std::lock_guard<std::mutex> lock(mutex_);
    if(out_ != nullptr) (*out_) << str << std::endl;
  }
 private:
  std::ostream* out_;
  std::mutex mutex_;
};
#endif
