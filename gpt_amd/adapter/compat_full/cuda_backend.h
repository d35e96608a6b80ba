// Name shim for the full-device build: the reference's gpt_test, train and
// infer sources construct their GPU backend by the class name CUDABackend
// (reference src/model/gpt_test.cpp:3, 219; src/train/train.cpp:2, 75;
// src/infer/infer.cpp:2, 80). Placed ahead of the reference's include
// directories, this header makes that name the all-GPU HIP backend
// (hip_backend.h: every op through the two C-ABI libraries), so those sources
// compile unchanged. It contains no CUDA API.
#pragma once

#include "hip_backend.h"

class CUDABackend : public HipBackend
{
public:
    explicit CUDABackend(unsigned long seed = 42) : HipBackend(seed) {}
};
