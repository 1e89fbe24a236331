// Measurement kernel: a plain streaming read, the ceiling a GEMV over the
// same bytes is measured against.  It has no counterpart in the reference.
//
// Every lane reads 16-byte pieces with nontemporal loads, P pieces a lane
// (1, 2 or 4, 1 KB apart inside a wave's span, the access width of the
// batch-1 GEMV kernels, and no arithmetic beyond an xor), so its time is
// the launch floor plus what the memory system delivers for those bytes.
#include "zt_common.h"

namespace zt {

template <int P>
__global__ void __launch_bounds__(256) stream_read_kernel(const uint4* __restrict__ p, long n16, uint32_t key,
                                                          uint32_t* __restrict__ sink) {
    const long base = (long)blockIdx.x * 256 * P + threadIdx.x;
    uint32_t acc = 0;
#pragma unroll
    for (int j = 0; j < P; j++) {
        const long i = base + 256 * j;
        if (i < n16) {
            const uint4 v = ld_stream(p + i);
            acc ^= v.x ^ v.y ^ v.z ^ v.w;
        }
    }
    if (acc == key) sink[0] = acc;  // keeps the loads; the key is chosen never to match in practice
}

}  // namespace zt

using namespace zt;

ZT_EXPORT int zt_bench_stream_read(const void* p, long nbytes, void* sink, hipStream_t stream) {
    if (nbytes < 0 || (nbytes > 0 && (p == nullptr || sink == nullptr)) || ((uintptr_t)p & 15))
        return (int)hipErrorInvalidValue;
    const long n16 = nbytes / 16;
    if (n16 == 0) return (int)hipSuccess;
    // pieces a lane: 4 while that leaves >= 2048 workgroups (8 waves a SIMD), else fewer, so small
    // buffers still spread over every CU
    const uint4* src = static_cast<const uint4*>(p);
    uint32_t* out = static_cast<uint32_t*>(sink);
    if (n16 >= 2048L * 1024)
        stream_read_kernel<4><<<ceil_div(n16, 1024), 256, 0, stream>>>(src, n16, 0x9E3779B9u, out);
    else if (n16 >= 2048L * 512)
        stream_read_kernel<2><<<ceil_div(n16, 512), 256, 0, stream>>>(src, n16, 0x9E3779B9u, out);
    else
        stream_read_kernel<1><<<ceil_div(n16, 256), 256, 0, stream>>>(src, n16, 0x9E3779B9u, out);
    return (int)hipGetLastError();
}
