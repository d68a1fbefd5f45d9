// Minimal Status / StatusOr with the numeric codes of absl::StatusCode, so
// the C-ABI returns the same code numbers the reference's absl::Status
// carries (e.g. InvalidArgument = 3, OutOfRange = 11).
#ifndef KVX_HOST_STATUS_H_
#define KVX_HOST_STATUS_H_

#include <optional>
#include <string>
#include <utility>

namespace kvx {

enum class Code : int {
  kOk = 0,
  kCancelled = 1,
  kUnknown = 2,
  kInvalidArgument = 3,
  kDeadlineExceeded = 4,
  kNotFound = 5,
  kAlreadyExists = 6,
  kPermissionDenied = 7,
  kResourceExhausted = 8,
  kFailedPrecondition = 9,
  kAborted = 10,
  kOutOfRange = 11,
  kUnimplemented = 12,
  kInternal = 13,
  kUnavailable = 14,
  kDataLoss = 15,
};

class Status {
 public:
  Status() = default;
  Status(Code code, std::string msg) : code_(code), msg_(std::move(msg)) {}
  bool ok() const { return code_ == Code::kOk; }
  Code code() const { return code_; }
  const std::string& message() const { return msg_; }
  std::string ToString() const;

 private:
  Code code_ = Code::kOk;
  std::string msg_;
};

inline Status OkStatus() { return Status(); }
inline Status InvalidArgumentError(std::string m) {
  return Status(Code::kInvalidArgument, std::move(m));
}
inline Status OutOfRangeError(std::string m) {
  return Status(Code::kOutOfRange, std::move(m));
}
inline Status FailedPreconditionError(std::string m) {
  return Status(Code::kFailedPrecondition, std::move(m));
}
inline Status ResourceExhaustedError(std::string m) {
  return Status(Code::kResourceExhausted, std::move(m));
}
inline Status InternalError(std::string m) {
  return Status(Code::kInternal, std::move(m));
}
inline Status NotFoundError(std::string m) {
  return Status(Code::kNotFound, std::move(m));
}
inline Status AlreadyExistsError(std::string m) {
  return Status(Code::kAlreadyExists, std::move(m));
}
inline Status CancelledError(std::string m) {
  return Status(Code::kCancelled, std::move(m));
}
inline Status UnimplementedError(std::string m) {
  return Status(Code::kUnimplemented, std::move(m));
}
inline Status DataLossError(std::string m) {
  return Status(Code::kDataLoss, std::move(m));
}
inline Status UnavailableError(std::string m) {
  return Status(Code::kUnavailable, std::move(m));
}

template <typename T>
class StatusOr {
 public:
  StatusOr(Status s) : status_(std::move(s)) {}  // NOLINT: implicit by design
  StatusOr(T v) : value_(std::move(v)) {}        // NOLINT: implicit by design
  bool ok() const { return status_.ok(); }
  const Status& status() const { return status_; }
  T& value() & { return *value_; }
  const T& value() const& { return *value_; }
  T&& value() && { return std::move(*value_); }
  T* operator->() { return &*value_; }
  T& operator*() { return *value_; }

 private:
  Status status_;
  std::optional<T> value_;
};

}  // namespace kvx

#define KVX_CONCAT_INNER(a, b) a##b
#define KVX_CONCAT(a, b) KVX_CONCAT_INNER(a, b)

#define KVX_RETURN_IF_ERROR(expr)          \
  do {                                     \
    ::kvx::Status _kvx_st = (expr);        \
    if (!_kvx_st.ok()) return _kvx_st;     \
  } while (0)

#define KVX_ASSIGN_OR_RETURN_IMPL(tmp, lhs, expr) \
  auto tmp = (expr);                              \
  if (!tmp.ok()) return tmp.status();             \
  lhs = std::move(tmp).value()

#define KVX_ASSIGN_OR_RETURN(lhs, expr) \
  KVX_ASSIGN_OR_RETURN_IMPL(KVX_CONCAT(_kvx_or_, __LINE__), lhs, expr)

#endif  // KVX_HOST_STATUS_H_
