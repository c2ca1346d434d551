/*
 * A stand-in libamdhip64.so.7 for CPU tests of libr9vx's failure paths: a
 * machine with the HIP runtime but no usable device.  It defines the HIP
 * entry points libr9vx imports (version node hip_4.2): registration of the
 * library's code objects succeeds, everything that needs a device fails
 * with hipErrorNoDevice (100) and leaves its outputs alone.  Built with
 * -DSTUB_WITHOUT_LAUNCH it lacks hipLaunchKernel, so loading libr9vx must
 * fail on the missing symbol.
 */
#include <stddef.h>
#include <stdint.h>

typedef int hipError_t;
typedef void *hipStream_t;
typedef struct {
    uint32_t x, y, z;
} dim3;

#define NO_DEVICE 100

static hipError_t last_error = 0;
static void *modules[4];

static hipError_t fail(void) {
    last_error = NO_DEVICE;
    return NO_DEVICE;
}

void **__hipRegisterFatBinary(const void *data) {
    (void)data;
    return modules;
}
void __hipUnregisterFatBinary(void **m) { (void)m; }
void __hipRegisterFunction(void **m, const void *host, char *dev, const char *name, unsigned limit, void *tid,
                           void *bid, void *bdim, void *gdim, int *wsize) {
    (void)m, (void)host, (void)dev, (void)name, (void)limit, (void)tid, (void)bid, (void)bdim, (void)gdim,
        (void)wsize;
}
void __hipRegisterVar(void **m, void *var, char *hvar, char *dvar, int ext, size_t size, int constant,
                      int global) {
    (void)m, (void)var, (void)hvar, (void)dvar, (void)ext, (void)size, (void)constant, (void)global;
}
hipError_t __hipPushCallConfiguration(dim3 g, dim3 b, size_t shmem, hipStream_t s) {
    (void)g, (void)b, (void)shmem, (void)s;
    return 0;
}
hipError_t __hipPopCallConfiguration(dim3 *g, dim3 *b, size_t *shmem, hipStream_t *s) {
    if (g) g->x = g->y = g->z = 1;
    if (b) b->x = b->y = b->z = 1;
    if (shmem) *shmem = 0;
    if (s) *s = 0;
    return 0;
}
#ifndef STUB_WITHOUT_LAUNCH
hipError_t hipLaunchKernel(const void *f, dim3 g, dim3 b, void **args, size_t shmem, hipStream_t s) {
    (void)f, (void)g, (void)b, (void)args, (void)shmem, (void)s;
    return fail();
}
#endif
hipError_t hipGetDevice(int *dev) {
    (void)dev;
    return fail();
}
hipError_t hipDeviceGetAttribute(int *v, int attr, int dev) {
    (void)v, (void)attr, (void)dev;
    return fail();
}
hipError_t hipGetLastError(void) {
    hipError_t e = last_error;
    last_error = 0;
    return e;
}
const char *hipGetErrorString(hipError_t e) { return e == NO_DEVICE ? "hipErrorNoDevice" : "stub error"; }
hipError_t hipGetSymbolAddress(void **p, const void *sym) {
    (void)p, (void)sym;
    return fail();
}
hipError_t hipMemcpyAsync(void *d, const void *s, size_t n, int kind, hipStream_t st) {
    (void)d, (void)s, (void)n, (void)kind, (void)st;
    return fail();
}
hipError_t hipMemcpy2DAsync(void *d, size_t dp, const void *s, size_t sp, size_t w, size_t h, int kind,
                            hipStream_t st) {
    (void)d, (void)dp, (void)s, (void)sp, (void)w, (void)h, (void)kind, (void)st;
    return fail();
}
hipError_t hipMemcpyFromSymbolAsync(void *d, const void *sym, size_t n, size_t off, int kind, hipStream_t st) {
    (void)d, (void)sym, (void)n, (void)off, (void)kind, (void)st;
    return fail();
}
hipError_t hipStreamSynchronize(hipStream_t s) {
    (void)s;
    return fail();
}
