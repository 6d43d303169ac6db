// Host-only stand-in for the HIP runtime API subset the transfer pipeline
// (stream-attn_amd/csrc/sa_pipeline.cpp) calls: types, constants and
// declarations only.  tests/native/fence_ledger.cpp defines the functions;
// they record every stream, event, copy and wait call in a ledger instead
// of touching a GPU, so the pipeline's ordering can be checked on a CPU.
#pragma once

#include <cstddef>
#include <cstdint>

typedef struct ihipStream_t* hipStream_t;
typedef struct ihipEvent_t* hipEvent_t;

enum hipError_t { hipSuccess = 0, hipErrorInvalidValue = 1, hipErrorNotReady = 600 };

enum hipMemcpyKind {
  hipMemcpyHostToHost = 0,
  hipMemcpyHostToDevice = 1,
  hipMemcpyDeviceToHost = 2,
  hipMemcpyDeviceToDevice = 3,
  hipMemcpyDefault = 4
};

#define hipStreamNonBlocking 0x01u
#define hipEventDisableTiming 0x02u

const char* hipGetErrorString(hipError_t error);
hipError_t hipGetDevice(int* device);
hipError_t hipSetDevice(int device);
hipError_t hipStreamCreateWithFlags(hipStream_t* stream, unsigned int flags);
hipError_t hipStreamDestroy(hipStream_t stream);
hipError_t hipStreamSynchronize(hipStream_t stream);
hipError_t hipStreamWaitEvent(hipStream_t stream, hipEvent_t event, unsigned int flags);
hipError_t hipEventCreate(hipEvent_t* event);
hipError_t hipEventCreateWithFlags(hipEvent_t* event, unsigned int flags);
hipError_t hipEventDestroy(hipEvent_t event);
hipError_t hipEventRecord(hipEvent_t event, hipStream_t stream);
hipError_t hipEventSynchronize(hipEvent_t event);
hipError_t hipEventElapsedTime(float* ms, hipEvent_t start, hipEvent_t stop);
hipError_t hipMemcpyAsync(void* dst, const void* src, size_t bytes, hipMemcpyKind kind, hipStream_t stream);
typedef void (*hipHostFn_t)(void* userData);
hipError_t hipLaunchHostFunc(hipStream_t stream, hipHostFn_t fn, void* userData);
hipError_t hipMemcpy2DAsync(void* dst, size_t dpitch, const void* src, size_t spitch, size_t width,
                             size_t height, hipMemcpyKind kind, hipStream_t stream);
