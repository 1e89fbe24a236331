/*
 * Calls libzt_hip.so the way the reference's zero-CGo binding does: one
 * dlopen, dlsym per entry point, and every call through a function pointer
 * cast to a 20-argument all-uintptr_t signature (cuda.Ccall,
 * internal/cuda/purego_linux_arm64_cgo.go:11-26 and
 * internal/cuda/purego_linux_arm64.go:47-112), with the result truncated to
 * the callee's int before it is compared, as a linux/amd64 trampoline must
 * (the SysV ABI leaves the upper half of RAX undefined for an int return).
 * Only argument-validation paths are called: every call returns before any
 * HIP runtime call, so no GPU is needed and no kernel is launched.
 *
 * The zero-CGo linux/amd64 binding resolves dlopen and dlsym as dynamic
 * imports of the executable and calls them through the same all-uintptr_t
 * trampoline as the entry points.  The first checks below do exactly that:
 * dlopen and dlsym are taken as plain addresses and called through the
 * 20-argument signature, and what they return must equal the direct calls.
 *
 * Usage: ccall_abi /path/to/libzt_hip.so   (exit status 0 = all checks pass)
 */
#define _GNU_SOURCE /* RTLD_DEFAULT */
#include <dlfcn.h>
#include <stdint.h>
#include <stdio.h>

typedef uintptr_t u;
typedef u (*ccall20)(u, u, u, u, u, u, u, u, u, u, u, u, u, u, u, u, u, u, u, u);

static void* lib;
static int failures;

static ccall20 sym(const char* name) {
    void* p = dlsym(lib, name);
    if (p == NULL) {
        printf("FAIL dlsym %s: %s\n", name, dlerror());
        failures++;
    }
    return (ccall20)p;
}

/* Ccall(fn, args...) with the unused argument slots zero, as the Go side
 * pads its [20]uintptr frame. */
static u call(ccall20 fn, u a0, u a1, u a2, u a3, u a4, u a5, u a6, u a7, u a8, u a9, u a10) {
    return fn(a0, a1, a2, a3, a4, a5, a6, a7, a8, a9, a10, 0, 0, 0, 0, 0, 0, 0, 0, 0);
}

static void expect_int(const char* what, u ret, int want) {
    const int got = (int)(int32_t)ret;
    if (got != want) {
        printf("FAIL %s: got %d, want %d\n", what, got, want);
        failures++;
    } else {
        printf("ok   %s = %d\n", what, got);
    }
}

static void expect_long(const char* what, u ret, long want) {
    if ((long)ret != want) {
        printf("FAIL %s: got %ld, want %ld\n", what, (long)ret, want);
        failures++;
    } else {
        printf("ok   %s = %ld\n", what, (long)ret);
    }
}

int main(int argc, char** argv) {
    if (argc != 2) {
        fprintf(stderr, "usage: %s libzt_hip.so\n", argv[0]);
        return 2;
    }
    lib = dlopen(argv[1], RTLD_NOW | RTLD_LOCAL);
    if (lib == NULL) {
        printf("FAIL dlopen: %s\n", dlerror());
        return 1;
    }
    /* dlopen and dlsym as addresses, called through the trampoline's signature */
    ccall20 dlopen_u = (ccall20)dlsym(RTLD_DEFAULT, "dlopen");
    ccall20 dlsym_u = (ccall20)dlsym(RTLD_DEFAULT, "dlsym");
    if (dlopen_u == NULL || dlsym_u == NULL) {
        printf("FAIL dlsym(RTLD_DEFAULT, dlopen/dlsym): %s\n", dlerror());
        return 1;
    }
    const u h = call(dlopen_u, (u)argv[1], RTLD_NOW | RTLD_GLOBAL, 0, 0, 0, 0, 0, 0, 0, 0, 0);
    expect_int("dlopen through the trampoline signature returns the library's handle", h == (u)lib, 1);
    const u fa = call(dlsym_u, h, (u) "zt_abi_version", 0, 0, 0, 0, 0, 0, 0, 0, 0);
    expect_int("dlsym through the trampoline signature finds zt_abi_version", fa == (u)dlsym(lib, "zt_abi_version"), 1);
    expect_int("dlsym through the trampoline signature of a missing name is 0",
               call(dlsym_u, h, (u) "zt_no_such_symbol", 0, 0, 0, 0, 0, 0, 0, 0, 0) == 0, 1);
    const u p = 0x100000; /* a 16-byte-aligned pointer value that is never dereferenced */
    const u neg1 = (u)(intptr_t)-1;

    ccall20 abi = sym("zt_abi_version");
    ccall20 q4 = sym("zt_gemm_q4_f32");
    ccall20 q8 = sym("zt_gemm_q8_f32");
    ccall20 tern = sym("zt_ternary_gemv_f32");
    ccall20 w4 = sym("zt_gemm_w4a16_f32");
    ccall20 q50t = sym("zt_gemm_q5_0t_f32");
    ccall20 grp = sym("zt_gemm_q4_group_f32");
    ccall20 off = sym("zt_q4_gpu_data_offset");
    ccall20 wsb = sym("zt_gemm_q4t_workspace_bytes");
    ccall20 w4sz = sym("zt_gemm_w4a16sz_f32");
    ccall20 w4t = sym("zt_gemm_w4a16t_f32");
    ccall20 w4tws = sym("zt_gemm_w4a16t_workspace_bytes");
    ccall20 iqt = sym("zt_gemm_iq4nlt_f16");
    ccall20 iqtws = sym("zt_gemm_iq4nlt_workspace_bytes");
    ccall20 tgrp = sym("zt_ternary_gemv_i8_group");
    ccall20 rd = sym("zt_bench_stream_read");
    ccall20 w4grp = sym("zt_gemv_w4a16sz_group_f32");
    if (failures) return 1;

    /* int return, no arguments */
    expect_int("zt_abi_version() / 100", call(abi, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0) / 100, 1);
    /* GemmQ4F32 with K % 32 != 0 -> InvalidValue (gemm_q4.cu:169-171), 8 arguments */
    expect_int("zt_gemm_q4_f32(K = 33)", call(q4, p, p, p, 4, 33, 1, 0, 0, 0, 0, 0), 1);
    /* negative sizes travel as sign-extended uintptr and arrive as int -1 */
    expect_int("zt_gemm_q4_f32(M = -1)", call(q4, p, p, p, neg1, 64, 1, 0, 0, 0, 0, 0), 1);
    /* M = 0 is a no-op success without touching the device */
    expect_int("zt_gemm_q4_f32(M = 0)", call(q4, p, p, p, 0, 64, 1, 0, 0, 0, 0, 0), 0);
    expect_int("zt_gemm_q8_f32(K = 48)", call(q8, p, p, p, 4, 48, 1, 0, 0, 0, 0, 0), 1);
    expect_int("zt_ternary_gemv_f32(null W)", call(tern, 0, p, p, 4, 16, 0, 0, 0, 0, 0, 0), 1);
    /* 10 arguments: group size not a multiple of 32 */
    expect_int("zt_gemm_w4a16_f32(group = 48)", call(w4, p, p, p, p, p, 4, 96, 1, 48, 0, 0), 1);
    /* 11 arguments, the largest arity: N = 5 is not a tiled batch */
    expect_int("zt_gemm_q5_0t_f32(N = 5)", call(q50t, p, p, p, p, p, 16, 128, 5, p, 4096, 0), 1);
    /* the batched W4A16 GEMM on packed scales: 9 arguments, N = 5 is not a batch it takes, M = 0 is a no-op */
    expect_int("zt_gemm_w4a16sz_f32(N = 5)", call(w4sz, p, p, p, p, 4, 128, 5, 128, 0, 0, 0), 1);
    expect_int("zt_gemm_w4a16sz_f32(M = 0)", call(w4sz, p, p, p, p, 0, 128, 4, 128, 0, 0, 0), 0);
    /* the tiled GEMMs take (workspace, workspace_bytes) before the stream: a split-K shape with no
       workspace is InvalidValue, and with the workspace it needs in the right argument slots the
       validation passes on to the size checks (a K that is not a multiple of 128 stays invalid) */
    expect_int("zt_gemm_w4a16t_workspace_bytes(1024, 8192, 8) > 0",
               (long)call(w4tws, 1024, 8192, 8, 0, 0, 0, 0, 0, 0, 0, 0) > 0, 1);
    expect_int("zt_gemm_w4a16t_f32(no workspace)", call(w4t, p, p, p, p, 1024, 8192, 8, 128, 0, 0, 0), 1);
    expect_int("zt_gemm_w4a16t_f32(M = 0, workspace slots)", call(w4t, p, p, p, p, 0, 8192, 8, 128, p, 1 << 20, 0), 0);
    expect_int("zt_gemm_iq4nlt_workspace_bytes(1024, 8192, 8) > 0",
               (long)call(iqtws, 1024, 8192, 8, 0, 0, 0, 0, 0, 0, 0, 0) > 0, 1);
    expect_int("zt_gemm_iq4nlt_f16(no workspace)", call(iqt, p, p, p, p, 1024, 8192, 8, 0, 0, 0, 0), 1);
    /* a host pointer argument: zero descriptors */
    expect_int("zt_gemm_q4_group_f32(n = 0)", call(grp, p, 0, p, 64, 0, 0, 0, 0, 0, 0, 0), 1);
    /* the grouped ternary GEMV reads its host descriptors before any launch: a matrix without
       weights is InvalidValue, every matrix empty is a no-op success */
    struct {
        u W, w_scale, y;
        int rows, reserved;
    } td[2] = {{0, p, p, 4, 0}, {0, 0, 0, 0, 0}};
    expect_int("zt_ternary_gemv_i8_group(no weights)", call(tgrp, (u)&td[0], 1, p, p, 64, 0, 0, 0, 0, 0, 0), 1);
    expect_int("zt_ternary_gemv_i8_group(all empty)", call(tgrp, (u)&td[1], 1, p, p, 64, 0, 0, 0, 0, 0, 0), 0);
    expect_int("zt_ternary_gemv_i8_group(n = 0)", call(tgrp, (u)&td[1], 0, p, p, 64, 0, 0, 0, 0, 0, 0), 1);
    /* the grouped W4A16 GEMV: host descriptors, a group size that is not a multiple of 32, all empty */
    struct {
        u W, szr, y;
        int rows, reserved;
    } wd[2] = {{p, p, p, 4, 0}, {0, 0, 0, 0, 0}};
    expect_int("zt_gemv_w4a16sz_group_f32(group = 48)", call(w4grp, (u)&wd[0], 1, p, 96, 48, 0, 0, 0, 0, 0, 0), 1);
    expect_int("zt_gemv_w4a16sz_group_f32(all empty)", call(w4grp, (u)&wd[1], 1, p, 128, 128, 0, 0, 0, 0, 0, 0), 0);
    /* the streaming-read measurement kernel: a long size argument, a misaligned buffer, an empty read */
    expect_int("zt_bench_stream_read(p + 8)", call(rd, p + 8, 4096, p, 0, 0, 0, 0, 0, 0, 0, 0), 1);
    expect_int("zt_bench_stream_read(nbytes = -1)", call(rd, p, neg1, p, 0, 0, 0, 0, 0, 0, 0, 0), 1);
    expect_int("zt_bench_stream_read(nbytes = 0)", call(rd, p, 0, p, 0, 0, 0, 0, 0, 0, 0, 0), 0);
    /* long returns come back whole */
    expect_long("zt_q4_gpu_data_offset(5)", call(off, 5, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0), 16);
    expect_long("zt_q4_gpu_data_offset(1<<31)", call(off, (u)1 << 31, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0), 1L << 32);
    expect_long("zt_gemm_q4t_workspace_bytes(K = 96)", call(wsb, 16, 96, 8, 0, 0, 0, 0, 0, 0, 0, 0), -1);

    dlclose(lib);
    if (failures) {
        printf("%d check(s) failed\n", failures);
        return 1;
    }
    printf("all checks passed\n");
    return 0;
}
