// tensorn_shim.hpp -- the slice of TensorN's tensor API that CXX-GPT's
// attention call sites use, backed by HIP device memory.
//
// TensorN (the reference's tensor library) is an un-vendored subproject; the
// attention path only touches CudaTensor<float>'s constructor from a shape,
// device_ptr(), shape(), size(), memset_zero(), copyFromHost(),
// fromTensor()/toTensor(), and host Tensor<float>(shape, vector) with a
// shared data vector and operator[] (uses at two_stage_cuda_kernels.cu:853,
// :1751, two_stage_gpt.hpp:105, :577, kernel_test.cpp:198, :225, :231).
// Include this header only where the real TensorN is absent.  It also
// provides the two macros of TensorN's that those call sites rely on,
// TENSORN_CUDA_AVAILABLE and CHECK_CUDA_ERROR.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <functional>
#include <memory>
#include <numeric>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#define CXG_HIP_CHECK(expr)                                                                  \
    do {                                                                                     \
        hipError_t cxg_e_ = (expr);                                                          \
        if (cxg_e_ != hipSuccess)                                                            \
            throw std::runtime_error(std::string("HIP error: ") + hipGetErrorString(cxg_e_) + \
                                     " at " + __FILE__ + ":" + std::to_string(__LINE__));    \
    } while (0)

// TensorN defines TENSORN_CUDA_AVAILABLE when it is built with its GPU
// backend; the reference's GPU call sites compile only under it
// (two_stage_gpt.hpp:7, linear_gpt.hpp:6, gpt_gpt.hpp:21).  This stand-in is
// the GPU backend, so it defines it.
#ifndef TENSORN_CUDA_AVAILABLE
#define TENSORN_CUDA_AVAILABLE 1
#endif

// TensorN's status check, used after launches as CHECK_CUDA_ERROR(<status>)
// (linear_cuda_kernels.cu:98, gpt_cuda_kernels.cu:30): here it takes a
// hipError_t (e.g. hipGetLastError()) and throws std::runtime_error naming the
// error and the call site when it is not hipSuccess.
#ifndef CHECK_CUDA_ERROR
#define CHECK_CUDA_ERROR(expr) CXG_HIP_CHECK(expr)
#endif

namespace TensorN {

inline size_t shape_numel(const std::vector<size_t>& s)
{
    return std::accumulate(s.begin(), s.end(), (size_t)1, std::multiplies<size_t>());
}

template <class T>
struct Tensor {
    std::vector<size_t> shape_;
    std::shared_ptr<std::vector<T>> data;

    Tensor(std::vector<size_t> shape, std::vector<T> values)
        : shape_(std::move(shape)), data(std::make_shared<std::vector<T>>(std::move(values)))
    {
        if (data->size() != shape_numel(shape_))
            throw std::invalid_argument("Tensor: value count does not match shape");
    }
    explicit Tensor(std::vector<size_t> shape)
        : Tensor(shape, std::vector<T>(shape_numel(shape)))
    {
    }
    const std::vector<size_t>& shape() const { return shape_; }
    size_t size() const { return data->size(); }
    T& operator[](size_t i) { return (*data)[i]; }
    const T& operator[](size_t i) const { return (*data)[i]; }
};

template <class T>
class CudaTensor {
public:
    explicit CudaTensor(std::vector<size_t> shape) : shape_(std::move(shape)), n_(shape_numel(shape_))
    {
        if (n_ > 0)
            CXG_HIP_CHECK(hipMalloc(&p_, n_ * sizeof(T)));
    }
    ~CudaTensor()
    {
        if (p_)
            (void)hipFree(p_);
    }
    CudaTensor(const CudaTensor&) = delete;
    CudaTensor& operator=(const CudaTensor&) = delete;
    CudaTensor(CudaTensor&& o) noexcept : shape_(std::move(o.shape_)), n_(o.n_), p_(o.p_)
    {
        o.p_ = nullptr;
        o.n_ = 0;
    }
    CudaTensor& operator=(CudaTensor&& o) noexcept
    {
        if (this != &o) {
            if (p_)
                (void)hipFree(p_);
            shape_ = std::move(o.shape_);
            n_ = o.n_;
            p_ = o.p_;
            o.p_ = nullptr;
            o.n_ = 0;
        }
        return *this;
    }

    T* device_ptr() const { return p_; }
    const std::vector<size_t>& shape() const { return shape_; }
    size_t size() const { return n_; }

    // stream-ordered on the legacy default stream, like the kernel launches
    void memset_zero()
    {
        if (n_)
            CXG_HIP_CHECK(hipMemsetAsync(p_, 0, n_ * sizeof(T), nullptr));
    }
    void copyFromHost(const T* src, size_t n)
    {
        if (n > n_)
            throw std::out_of_range("CudaTensor::copyFromHost: too many elements");
        if (n)
            CXG_HIP_CHECK(hipMemcpy(p_, src, n * sizeof(T), hipMemcpyHostToDevice));
    }
    static CudaTensor fromTensor(const Tensor<T>& t)
    {
        CudaTensor c(t.shape());
        c.copyFromHost(t.data->data(), t.size());
        return c;
    }
    Tensor<T> toTensor() const
    {
        Tensor<T> t(shape_);
        if (n_)
            CXG_HIP_CHECK(hipMemcpy(t.data->data(), p_, n_ * sizeof(T), hipMemcpyDeviceToHost));
        return t;
    }

private:
    std::vector<size_t> shape_;
    size_t n_ = 0;
    T* p_ = nullptr;
};

} // namespace TensorN
