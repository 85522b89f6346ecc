// qr_host.cpp -- the bridge's host-only logic: argument validation and the
// host-range probe.  No HIP calls, so a sanitizer build of the host code can
// compile it alone (tests/c/sanitize_host.cpp).
#include "qr_host.h"

#include <sys/uio.h>
#include <unistd.h>

#include <cerrno>

namespace qr {

// Whether every page of the host range [p, p + bytes) can be read (and, for
// outputs, written) by this process.  The reference wraps host memory with
// newBufferWithBytesNoCopy and returns -5 when that fails for a range running
// into an unmapped or protected page (tests/redteam_bridge.py:178-221); here
// the staging copy would fault instead, so the range is probed first, one
// byte per page, by system calls that report EFAULT rather than raise a
// signal: process_vm_readv / process_vm_writev on this process, or where
// those are not permitted (seccomp), a pipe -- write(2) from the page reads
// it, read(2) of that byte back into the page writes it unchanged.  When no
// probe is possible the range counts as inaccessible (fail closed: -5).
static bool page_ok_pipe(int fds[2], const void* q, bool write) {
    char sink;
    if (::write(fds[1], q, 1) != 1) return false;  // EFAULT: not readable
    if (write) {
        if (::read(fds[0], const_cast<void*>(q), 1) == 1) return true;
        (void)::read(fds[0], &sink, 1);  // not writable: drain the byte
        return false;
    }
    return ::read(fds[0], &sink, 1) == 1;
}

bool host_range_ok(const void* p, size_t bytes, bool write) {
    if (bytes == 0) return true;
    const uintptr_t pg = (uintptr_t)sysconf(_SC_PAGESIZE);
    const uintptr_t a = reinterpret_cast<uintptr_t>(p), e = a + bytes - 1;
    constexpr int kBatch = 512;
    char tmp[kBatch];
    struct iovec loc[kBatch], rem[kBatch];
    // probe addresses: a, then the first byte of every later page up to e
    uintptr_t q = a;
    bool more = true;
    while (more) {
        int n = 0;
        for (; n < kBatch && more; n++) {
            loc[n] = {tmp + n, 1};
            rem[n] = {reinterpret_cast<void*>(q), 1};
            const uintptr_t next = (q / pg + 1) * pg;
            more = next > q && next <= e;
            q = next;
        }
        errno = 0;
        ssize_t got = process_vm_readv(getpid(), loc, n, rem, n, 0);
        if (got >= 0 || errno == EFAULT) {
            if (got != n) return false;
            if (write) {
                got = process_vm_writev(getpid(), loc, n, rem, n, 0);  // the bytes just read, unchanged
                if (got != n) return false;
            }
            continue;
        }
        // process_vm_* not permitted: probe this batch's pages through a pipe
        int fds[2];
        if (pipe(fds) != 0) return false;
        bool ok = true;
        for (int i = 0; i < n && ok; i++) ok = page_ok_pipe(fds, rem[i].iov_base, write);
        close(fds[0]);
        close(fds[1]);
        if (!ok) return false;
    }
    return true;
}


// Formats m4_bridge_dispatch_gemm accepts (m4_mlx_bridge.mm:28-35, 211), and
// the wider set the kernel-name entry points accept: every format with a
// kernel here, i.e. also Q8_0 weights (6), PRISM_Q2_0 (7) and MLX g64 (8).
bool is_projection_format(int f) { return f >= 0 && f < 6; }
bool has_kernels(int f) { return f >= 0 && f <= qr::QUANT_MLX_4BIT_G64; }

// core/bridge/m4_mlx_bridge.mm:204-230, minus the init check.  `ext` widens
// the format range to every format with kernels (PRISM_Q2_0 needs K % 128).
int validate(const void* X, size_t Xb, const void* W, size_t Wb, const void* Y, size_t Yb, int format,
             uint32_t M, uint32_t K, uint32_t N, bool ext) {
    if (!X || !W || !Y) return -2;
    if ((reinterpret_cast<uintptr_t>(X) % 2) || (reinterpret_cast<uintptr_t>(Y) % 2)) return -2;
    if (!(ext ? has_kernels(format) : is_projection_format(format))) return -3;
    if (M == 0 || K == 0 || N == 0) return -4;
    if (K % 32) return -4;
    if ((format == 2 || format == 4 || format == 5) && (K % 256)) return -4;
    if (format == 7 && (K % 128)) return -4;
    if (format == qr::QUANT_MLX_4BIT_G64 && (K % 64)) return -4;
    if (Xb < (size_t)M * K * 2 || Yb < (size_t)M * N * 2 || Wb < qr::kernel_weight_bytes(format, K, N))
        return -2;
    return 0;
}

}  // namespace qr
