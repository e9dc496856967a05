// HIP error handling of the KV-cache path.  HIP_CHECK throws HipException,
// the counterpart of the reference's CUDA_CHECK / CudaException
// (include/tiny_llm/cuda_utils.h:14-20, 47-68): runtime failures inside
// appendKV surface as exceptions, host validation as Result::err.
#pragma once

#include <hip/hip_runtime_api.h>

#include <exception>
#include <string>

namespace tiny_llm {

class HipException : public std::exception {
  public:
    HipException(hipError_t err, const char *file, int line)
        : error_(err), file_(file), line_(line),
          message_("HIP error " + std::to_string(static_cast<int>(err)) + " at " + file + ":" +
                   std::to_string(line) + ": " + hipGetErrorString(err)) {}
    const char *what() const noexcept override { return message_.c_str(); }
    hipError_t  error() const { return error_; }
    const char *file() const { return file_; }
    int         line() const { return line_; }

  private:
    hipError_t  error_;
    const char *file_;
    int         line_;
    std::string message_;
};

} // namespace tiny_llm

#define HIP_CHECK(call)                                                                            \
    do {                                                                                           \
        hipError_t hip_check_err_ = (call);                                                        \
        if (hip_check_err_ != hipSuccess)                                                          \
            throw ::tiny_llm::HipException(hip_check_err_, __FILE__, __LINE__);                    \
    } while (0)
