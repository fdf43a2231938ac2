// Error and logging convention shared by every hot-path operator.
//
// Operators report failures by throwing rpg::Error; the C-ABI layer (capi.cc)
// catches it and turns it into a negative status plus a thread-local message,
// so no C++ exception ever crosses an extern "C" boundary.
//
// Interface kept alike on purpose (same names and meaning as the engine code that
// calls these operators): rpg::Error / rpg::Throw / RPG_CHECK / SetLastError /
// LastError follow src/common.h:22-58 and src/common.cc:54-66 of the reference.
#ifndef RPG_AMD_COMMON_H_
#define RPG_AMD_COMMON_H_

#include <stdexcept>
#include <string>

namespace rpg {

class Error : public std::runtime_error {
 public:
  explicit Error(const std::string& msg) : std::runtime_error(msg) {}
};

// Thread-local text of the most recent failure on this thread.
void SetLastError(const std::string& msg);
const char* LastError();

// printf-style formatting, records the text as the last error, then throws Error.
[[noreturn]] __attribute__((format(printf, 1, 2))) void Throw(const char* fmt, ...);

enum class LogLevel { kDebug, kInfo, kWarn, kError };
// Logging goes to stderr with a fixed prefix. RPGBAR_ENGINE_LOG selects the
// minimum level (debug/info/warn/error) or silences everything (off/0/false).
bool LogEnabled(LogLevel lv);
__attribute__((format(printf, 2, 3))) void Log(LogLevel lv, const char* fmt, ...);

}  // namespace rpg

// Argument check that is always on: a violated precondition throws rpg::Error.
#define RPG_CHECK(cond, ...)                    \
  do {                                          \
    if (!(cond)) ::rpg::Throw(__VA_ARGS__);     \
  } while (0)

#define RPG_LOG_INFO(...) ::rpg::Log(::rpg::LogLevel::kInfo, __VA_ARGS__)
#define RPG_LOG_WARN(...) ::rpg::Log(::rpg::LogLevel::kWarn, __VA_ARGS__)

#endif  // RPG_AMD_COMMON_H_
