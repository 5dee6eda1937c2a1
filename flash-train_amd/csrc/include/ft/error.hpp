// Status + message carried across the C ABI.
//
// Behaviour follows the reference's Result/Exception
// (src/include/flash_train/error.hpp:19-81, src/error.cpp:10-61): a message
// holds at most 2047 characters plus the terminator, a success never carries
// a message, and an Exception can never hold a success status.
#pragma once

#include <cstdarg>
#include <cstddef>
#include <exception>

#include <flash_train/common.h>

namespace ftrain {

class Result {
  public:
    static constexpr std::size_t kCapacity = 8192;  // bytes including the terminator (room for every variant's reason)

    Result() noexcept { text_[0] = '\0'; }
    Result(FTrainStatus status, const char* message) noexcept { set(status, message); }

    // Copies `message` verbatim (no formatting), truncated to kCapacity - 1.
    void set(FTrainStatus status, const char* message) noexcept;
    // printf-style; a formatting error keeps the status with an empty message.
    void format(FTrainStatus status, const char* fmt, ...) noexcept __attribute__((format(printf, 3, 4)));
    void vformat(FTrainStatus status, const char* fmt, std::va_list args) noexcept;
    void clear() noexcept {
        status_  = FTRAIN_STATUS_SUCCESS;
        text_[0] = '\0';
    }

    bool isSuccess() const noexcept { return status_ == FTRAIN_STATUS_SUCCESS; }
    FTrainStatus getStatus() const noexcept { return status_; }
    const char* getMessage() const noexcept { return text_; }

  private:
    FTrainStatus status_ = FTRAIN_STATUS_SUCCESS;
    char text_[kCapacity];
};

class Exception final : public std::exception {
  public:
    explicit Exception(const Result& result) noexcept;
    Exception(FTrainStatus status, const char* fmt, ...) noexcept __attribute__((format(printf, 3, 4)));

    const Result& getResult() const noexcept { return result_; }
    const char* what() const noexcept override { return result_.getMessage(); }

  private:
    Result result_;
};

}  // namespace ftrain
