// hip_check.hpp -- error conventions of the host layer: every HIP or libsgq
// failure becomes std::runtime_error naming the call and its file:line, as the
// reference's CUDA_CHECK does (include/sovereigngrad/cuda_mock.hpp:149-155).
#pragma once

#include <hip/hip_runtime_api.h>

#include <stdexcept>
#include <string>

#include "sgq.h"

#define SG_HIP_CHECK(expr)                                                                                   \
    do {                                                                                                     \
        hipError_t sg_err_ = (expr);                                                                         \
        if (sg_err_ != hipSuccess)                                                                           \
            throw std::runtime_error(std::string("HIP error: ") + hipGetErrorString(sg_err_) + " (" #expr ") at " + \
                                     __FILE__ + ":" + std::to_string(__LINE__));                             \
    } while (0)

#define SG_SGQ_CHECK(expr)                                                                                   \
    do {                                                                                                     \
        int sg_st_ = (expr);                                                                                 \
        if (sg_st_ != SGQ_OK)                                                                                \
            throw std::runtime_error(std::string("libsgq error ") + std::to_string(sg_st_) + ": " +          \
                                     sgq_last_error() + " (" #expr ") at " + __FILE__ + ":" +                \
                                     std::to_string(__LINE__));                                              \
    } while (0)
