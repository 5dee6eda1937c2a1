// Status + message carried across the C ABI.
//
// The observable contract is the reference's (src/include/flash_train/error.hpp:17-81):
// a message holds at most 2047 characters plus the terminator, a success
// never carries a message, and a failure raised with a success status
// surfaces as INTERNAL_ERROR.  Inside the library a failure is raised with
// raise() and caught once, at the C entry point (handles.hpp), which moves
// its Result into the calling thread's last-result slot.
#pragma once

#include <array>
#include <cstdarg>
#include <cstddef>
#include <exception>

#include <flash_train/common.h>

namespace ftrain {

class Result {
  public:
    // Bytes of message storage, terminator included (reference error.hpp:52).
    static constexpr std::size_t kMessageBytes = 2048;

    Result() noexcept = default;
    Result(FTrainStatus status, const char* message) noexcept { set(status, message); }

    // Stores `message` as literal text; a success or null message stores "".
    void set(FTrainStatus status, const char* message) noexcept { compose(status, message, nullptr); }
    // printf-style; a formatting error keeps the status with an empty message.
    void format(FTrainStatus status, const char* fmt, ...) noexcept __attribute__((format(printf, 3, 4)));
    void vformat(FTrainStatus status, const char* fmt, std::va_list args) noexcept;
    void clear() noexcept { compose(FTRAIN_STATUS_SUCCESS, nullptr, nullptr); }

    bool isSuccess() const noexcept { return status_ == FTRAIN_STATUS_SUCCESS; }
    FTrainStatus getStatus() const noexcept { return status_; }
    const char* getMessage() const noexcept { return text_.data(); }

  private:
    // One writer for every setter: `args` null means `text` is literal.
    void compose(FTrainStatus status, const char* text, std::va_list* args) noexcept;

    FTrainStatus status_ = FTRAIN_STATUS_SUCCESS;
    std::array<char, kMessageBytes> text_{};
};

// The one exception type the library throws; it owns a failed Result.
class Failure final : public std::exception {
  public:
    explicit Failure(const Result& result) noexcept;

    const Result& result() const noexcept { return result_; }
    const char* what() const noexcept override { return result_.getMessage(); }

  private:
    Result result_;
};

// Throws a Failure with the formatted message.
[[noreturn]] void raise(FTrainStatus status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

}  // namespace ftrain
