// hip_device.h - HipDevice: the expert store's device backend on MI355X,
// built only on libeahmmf_hip.so's C ABI (no HIP headers needed).
//
// The reference's expert store programs against DeviceBackend
// (eahmmf.h:88-100); its CUDA implementation is CudaDevice (eahmmf.h:150-200).
// HipDeviceOn<Base> implements that interface over any base class with the
// same virtual methods:
//   - inside the reference build:  HipDeviceOn<eahmmf::DeviceBackend>
//   - standalone (this repository): HipDevice = HipDeviceOn<DeviceBackend>
//     with the interface restated below.
// Semantics kept from CudaDevice:
//   total_memory()  free device memory at construction
//   free_memory()   physical free memory now (hipMemGetInfo), 0 on error
//   alloc()         nullptr on failure, with a one-line diagnostic on stderr
//   h2d()           asynchronous on the library's stream (valid after sync())
//   d2h()           synchronous
//   cpu_readable()  false: CPU kernels cannot dereference device pointers
// The library's expert kernels run on the same per-device stream, so an
// expert staged with h2d() is visible to the next synchronous call.
#ifndef EAHMMF_HIP_DEVICE_H
#define EAHMMF_HIP_DEVICE_H
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>

#include "eahmmf_hip.h"

namespace eahmmf_hip {

// The device-backend interface of the reference's expert store
// (eahmmf.h:88-100): same method names, arguments and meaning.
struct DeviceBackend {
    virtual ~DeviceBackend() {}
    virtual const char* name() const = 0;
    virtual void* alloc(size_t bytes) = 0;  // nullptr on failure
    virtual void release(void* p, size_t bytes) = 0;
    virtual bool h2d(void* dev_dst, const void* host_src, size_t n) = 0;
    virtual bool d2h(void* host_dst, const void* dev_src, size_t n) = 0;
    virtual bool sync() = 0;  // copies are valid for compute only after sync()
    virtual bool cpu_readable() const = 0;
    virtual size_t total_memory() const { return SIZE_MAX; }
    virtual size_t free_memory() const { return SIZE_MAX; }
};

template <class Base>
struct HipDeviceOn : Base {
    size_t total = 0;
    HipDeviceOn() {
        size_t fr = 0, tot = 0;
        if (eahmmf_hip_mem_info(&fr, &tot) == 0) total = fr;
    }
    const char* name() const override { return "hip"; }
    void* alloc(size_t n) override {
        void* p = nullptr;
        if (eahmmf_hip_alloc(&p, n) != 0 || !p) {
            size_t fr = 0, tot = 0;
            const bool have = eahmmf_hip_mem_info(&fr, &tot) == 0;
            fprintf(stderr, "[EAHMMF HIP] device allocation failed: requested=%zu bytes (%s), free=%zu MiB, total=%zu MiB\n",
                    n, eahmmf_hip_last_error(), have ? fr >> 20 : (size_t)0, have ? tot >> 20 : (size_t)0);
            return nullptr;
        }
        return p;
    }
    void release(void* p, size_t) override {
        if (p) (void)eahmmf_hip_free(p);
    }
    bool h2d(void* d, const void* s, size_t n) override { return eahmmf_hip_h2d(d, s, n) == 0; }
    bool d2h(void* d, const void* s, size_t n) override { return eahmmf_hip_d2h(d, s, n) == 0; }
    bool sync() override { return eahmmf_hip_sync() == 0; }
    // Not in the reference's interface: many host-to-device copies in one
    // call through the library's pinned staging ring (valid for compute when
    // it returns), for preloading experts instead of one h2d() + sync() each.
    bool h2d_batch(const eahmmf_hip_copy* copies, int n) { return eahmmf_hip_h2d_batch(copies, n) == 0; }
    // Not in the reference's interface either: the same batch queued to the
    // library's staging thread (asynchronous prefetch, which the reference
    // lists as not implemented, README.md:379).  Returns a ticket (0 on
    // failure); the sources must stay valid until h2d_batch_wait(ticket)
    // has returned true.  With a stream, work queued on it afterwards waits
    // on the device for the bytes; without, the host waits until they land.
    uint64_t h2d_batch_async(const eahmmf_hip_copy* copies, int n) {
        uint64_t t = 0;
        return eahmmf_hip_h2d_batch_async(copies, n, &t) == 0 ? t : 0;
    }
    bool h2d_batch_wait(uint64_t ticket, void* stream = nullptr) {
        return eahmmf_hip_h2d_batch_wait(ticket, stream) == 0;
    }
    bool cpu_readable() const override { return false; }
    size_t total_memory() const override { return total; }
    size_t free_memory() const override {
        size_t fr = 0, tot = 0;
        return eahmmf_hip_mem_info(&fr, &tot) == 0 ? fr : 0;
    }
};

using HipDevice = HipDeviceOn<DeviceBackend>;

}  // namespace eahmmf_hip
#endif
