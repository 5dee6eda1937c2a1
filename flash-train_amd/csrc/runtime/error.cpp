#include "ft/error.hpp"

#include <cstdio>
#include <cstring>

namespace ftrain {

namespace {
constexpr const char* kSuccessException = "Exception cannot be constructed with FTRAIN_STATUS_SUCCESS";
}

void Result::set(FTrainStatus status, const char* message) noexcept {
    status_  = status;
    text_[0] = '\0';
    if (status == FTRAIN_STATUS_SUCCESS || message == nullptr) return;
    const std::size_t n = strnlen(message, kCapacity - 1);
    std::memcpy(text_, message, n);
    text_[n] = '\0';
}

void Result::vformat(FTrainStatus status, const char* fmt, std::va_list args) noexcept {
    status_  = status;
    text_[0] = '\0';
    if (status == FTRAIN_STATUS_SUCCESS || fmt == nullptr) return;
    if (std::vsnprintf(text_, kCapacity, fmt, args) < 0) text_[0] = '\0';
    text_[kCapacity - 1] = '\0';
}

void Result::format(FTrainStatus status, const char* fmt, ...) noexcept {
    std::va_list args;
    va_start(args, fmt);
    vformat(status, fmt, args);
    va_end(args);
}

Exception::Exception(const Result& result) noexcept : result_(result) {
    if (result_.isSuccess()) result_.set(FTRAIN_STATUS_INTERNAL_ERROR, kSuccessException);
}

Exception::Exception(FTrainStatus status, const char* fmt, ...) noexcept {
    if (status == FTRAIN_STATUS_SUCCESS) {
        result_.set(FTRAIN_STATUS_INTERNAL_ERROR, kSuccessException);
        return;
    }
    std::va_list args;
    va_start(args, fmt);
    result_.vformat(status, fmt, args);
    va_end(args);
}

}  // namespace ftrain
