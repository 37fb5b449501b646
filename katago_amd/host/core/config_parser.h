// Stand-in for KataGo's cpp/core/config_parser.h: the key/value config a
// backend may consult for its own options (nninterface.h:56-58).
#ifndef KATAGO_AMD_CORE_CONFIG_PARSER_H
#define KATAGO_AMD_CORE_CONFIG_PARSER_H
#include <map>
#include <string>
#include "global.h"

class ConfigParser {
 public:
  ConfigParser() = default;
  void overrideKey(const std::string& key, const std::string& value) { kv_[key] = value; }
  bool contains(const std::string& key) const { return kv_.find(key) != kv_.end(); }
  std::string getString(const std::string& key) const {
    auto it = kv_.find(key);
    if(it == kv_.end()) throw StringError("Could not find key '" + key + "' in config");
    return it->second;
  }
  bool getBool(const std::string& key) const {
    std::string v = getString(key);
    if(v == "true" || v == "1" || v == "yes") return true;
    if(v == "false" || v == "0" || v == "no") return false;
    throw StringError("Could not parse '" + v + "' as bool for key '" + key + "'");
  }
  int getInt(const std::string& key) const {
    std::string v = getString(key);
    try { return std::stoi(v); } catch(...) { throw StringError("Could not parse '" + v + "' as int for key '" + key + "'"); }
  }
 private:
  std::map<std::string, std::string> kv_;
};
#endif
