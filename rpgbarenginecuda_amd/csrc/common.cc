// Implementation of the error / logging convention declared in common.h.
#include "common.h"

#include <cctype>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>

namespace rpg {
namespace {

thread_local std::string t_last_error;

const char* LevelTag(LogLevel lv) {
  switch (lv) {
    case LogLevel::kDebug: return "debug";
    case LogLevel::kInfo: return "info";
    case LogLevel::kWarn: return "warn";
    case LogLevel::kError: return "error";
  }
  return "?";
}

// Parsed once: the environment is read at the first log call.
struct LogConfig {
  bool off = false;
  LogLevel min = LogLevel::kInfo;
};

const LogConfig& Config() {
  static const LogConfig cfg = [] {
    LogConfig c;
    const char* v = std::getenv("RPGBAR_ENGINE_LOG");
    if (v == nullptr) return c;
    std::string s(v);
    for (char& ch : s) ch = static_cast<char>(std::tolower(static_cast<unsigned char>(ch)));
    if (s == "off" || s == "0" || s == "false") c.off = true;
    else if (s == "debug") c.min = LogLevel::kDebug;
    else if (s == "warn") c.min = LogLevel::kWarn;
    else if (s == "error") c.min = LogLevel::kError;
    return c;
  }();
  return cfg;
}

}  // namespace

void SetLastError(const std::string& msg) { t_last_error = msg; }

const char* LastError() { return t_last_error.c_str(); }

void Throw(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  SetLastError(buf);
  throw Error(std::string(buf));
}

bool LogEnabled(LogLevel lv) {
  const LogConfig& c = Config();
  return !c.off && static_cast<int>(lv) >= static_cast<int>(c.min);
}

void Log(LogLevel lv, const char* fmt, ...) {
  if (!LogEnabled(lv)) return;
  char buf[2048];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  static std::mutex mu;
  std::lock_guard<std::mutex> lk(mu);
  std::fprintf(stderr, "[rpg_engine %s] %s\n", LevelTag(lv), buf);
  std::fflush(stderr);
}

}  // namespace rpg
