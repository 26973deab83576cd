// extern "C" boundary of libfoundry_attn.so (declared in include/foundry_attn.h).
// Validates every argument before touching the device, maps failures to
// fa_status codes with a thread-local message, and forwards to the kernel
// launchers.  No C++ exception crosses the boundary.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "../../include/foundry_attn.h"
#include "../../include/foundry_block.h"
#include "fa_kernels.hpp"

// Scratch of fa_attn_bwd_noalloc: the backward's delta and lse2 rows
// ([B,H,S] f32 each, 256-byte aligned), FA_BWD_NOALLOC_MAX_ROWS rows apiece.
// Every GPU holds its own copy for the life of the process, and every call on
// one GPU shares it.  On the host `scratch` names a host-side stand-in, not
// device memory: kernels and copies get the per-device address that
// setup_scratch_locked looks up (g_scratch), never the array's name.
static __device__ __align__(256) unsigned char scratch[FA_BWD_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local char g_err[512] = "";

fa_status fail(fa_status code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

fa_status ok() {
    g_err[0] = '\0';
    return FA_OK;
}

constexpr int kMaxDevices = 64;
std::mutex g_init_mu;
int g_dev_state[kMaxDevices];  // 0 unknown, 1 ready, -1 unsupported
bool g_prepared = false;

fa_status hip_fail(hipError_t e, const char *what) {
    return fail(FA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

constexpr int kNoallocScratchBytes = FA_BWD_NOALLOC_SCRATCH_BYTES;
void *g_scratch[kMaxDevices];  // device address of `scratch` per device (under g_init_mu)

bool aligned_ptr(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

fa_status init_device(int device) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0)
        return fail(FA_ERR_NO_DEVICE, "no HIP device visible");
    if (device < 0 || device >= count || device >= kMaxDevices)
        return fail(FA_ERR_INVALID_ARG, "device %d out of range (count %d)", device, count);
    std::lock_guard<std::mutex> lk(g_init_mu);
    if (g_dev_state[device] == 0) {
        hipDeviceProp_t prop;
        hipError_t e = hipGetDeviceProperties(&prop, device);
        if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
        g_dev_state[device] = strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : -1;
        if (g_dev_state[device] < 0)
            return fail(FA_ERR_LOAD_FAILED, "device %d is %s; this library holds gfx950 code only",
                        device, prop.gcnArchName);
    }
    if (g_dev_state[device] < 0) return fail(FA_ERR_LOAD_FAILED, "device %d is not gfx950", device);
    if (!g_prepared) {
        hipError_t e = fa::prepare_attn_kernels();
        if (e != hipSuccess) return hip_fail(e, "kernel attribute setup");
        g_prepared = true;
    }
    return FA_OK;
}

fa_status init_current() {
    int dev = 0, count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0)
        return fail(FA_ERR_NO_DEVICE, "no HIP device visible");
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    return init_device(dev);
}

bool aligned(const void *p, size_t a) { return aligned_ptr(p, a); }

// Looks up, once per device, the device address of the no-allocation scratch
// (each GPU holds its own copy of `scratch` at its own address) with `device`
// current; only fa_init and fa_attn_bwd_noalloc need it.  Caller holds
// g_init_mu.
fa_status setup_scratch_locked(int device) {
    if (g_scratch[device]) return FA_OK;
    int cur = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (cur != device && (e = hipSetDevice(device)) != hipSuccess) return hip_fail(e, "hipSetDevice");
    void *ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    const hipError_t e2 = cur != device ? hipSetDevice(cur) : hipSuccess;
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (e2 != hipSuccess) return hip_fail(e2, "hipSetDevice (restore)");
    if (!ptr || !aligned_ptr(ptr, 256)) return fail(FA_ERR_HIP, "no-allocation scratch is misaligned");
    g_scratch[device] = ptr;
    return FA_OK;
}

// Device address of the no-allocation scratch on the current device, looked
// up on first use there unless fa_init(device) already did.
fa_status scratch_for_current(char **out) {
    int dev = 0;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return fail(FA_ERR_INVALID_ARG, "device %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_init_mu);
    const fa_status st = setup_scratch_locked(dev);
    if (st != FA_OK) return st;
    *out = static_cast<char *>(g_scratch[dev]);
    return FA_OK;
}

const char *dtype_name(int32_t dt) { return dt == FA_DTYPE_BF16 ? "bf16" : "f32"; }

// Checks a [B,S,H,D] view: non-null, non-negative strides, and every row
// start 16-byte aligned (the kernels move rows with 16-byte vector loads):
// base pointer 16-byte aligned, strides multiples of 8 (bf16) or 4 (f32)
// elements.
fa_status check_view(const char *name, const void *ptr, const fa_strides &st, int32_t dtype) {
    if (!ptr) return fail(FA_ERR_INVALID_ARG, "%s is NULL", name);
    if (st.b < 0 || st.s < 0 || st.h < 0)
        return fail(FA_ERR_INVALID_ARG, "%s has a negative stride", name);
    const int64_t mult = dtype == FA_DTYPE_BF16 ? 8 : 4;
    if (!aligned(ptr, 16)) return fail(FA_ERR_INVALID_ARG, "%s is not 16-byte aligned", name);
    if (st.b % mult || st.s % mult || st.h % mult)
        return fail(FA_ERR_INVALID_ARG,
                    "%s strides (%lld,%lld,%lld) must be multiples of %lld elements (%s)", name,
                    (long long)st.b, (long long)st.s, (long long)st.h, (long long)mult,
                    dtype_name(dtype));
    return FA_OK;
}

fa_status check_attn_shape(int32_t dtype, int32_t B, int32_t S, int32_t H, int32_t D, float scale) {
    if (dtype != FA_DTYPE_BF16 && dtype != FA_DTYPE_F32)
        return fail(FA_ERR_INVALID_ARG, "unknown dtype %d", dtype);
    if (B < 1 || S < 1 || H < 1)
        return fail(FA_ERR_INVALID_ARG, "batch/seq/heads must be >= 1 (got %d/%d/%d)", B, S, H);
    if (S > (1 << 22)) return fail(FA_ERR_INVALID_ARG, "seq %d exceeds 4194304", S);
    if (D != 64 && D != 128)
        return fail(FA_ERR_UNSUPPORTED, "head_dim %d: this build implements 64 and 128", D);
    if (!isfinite(scale) || !(scale > 0.f))
        return fail(FA_ERR_INVALID_ARG, "scale must be finite and > 0 (got %g)", (double)scale);
    const int64_t tiles = (int64_t)B * H * ((S + 31) / 32);
    if (tiles > 0x7fffffffLL) return fail(FA_ERR_INVALID_ARG, "B*H*S too large for one launch");
    return FA_OK;
}

// The bf16 kernels address K/V (and the backward's Q/dO) through 32-bit
// buffer offsets and rely on rows of one head not overlapping, so rows past S
// fall outside the buffer range and read as zero.
fa_status check_buffer_view(const char *name, const fa_strides &st, int32_t S, int32_t D) {
    if (st.s < D)
        return fail(FA_ERR_INVALID_ARG, "%s sequence stride %lld is smaller than head_dim %d", name,
                    (long long)st.s, D);
    const int64_t bytes = ((int64_t)(S - 1) * st.s + D) * 2 + (int64_t)64 * st.s * 2;
    if (bytes >= (int64_t(1) << 31))
        return fail(FA_ERR_UNSUPPORTED, "%s spans %lld bytes per head; this build addresses < 2 GiB",
                    name, (long long)bytes);
    return FA_OK;
}

size_t round256(size_t x) { return (x + 255) & ~size_t(255); }

// Range split factor of a bf16 call (1 for f32 or unsplit shapes).
int split_for(int32_t dtype, int32_t B, int32_t S, int32_t H) {
    return dtype == FA_DTYPE_BF16 ? fa::attn_split(B, H, S) : 1;
}

// backward workspace: delta [B,H,S] f32, lse2 [B,H,S] f32, then for a split
// call the f32 partials of dQ, dK and dV ([split][B,H,S][D] each).  This much
// runs the backward that recomputes S and dP in the dQ kernel.
size_t bwd_min_workspace(int32_t dtype, int32_t B, int32_t S, int32_t H, int32_t D) {
    const int split = split_for(dtype, B, S, H);
    return 2 * round256((size_t)B * H * S * sizeof(float)) +
           3 * round256(fa::attn_split_elems(B, H, S, D, split) * sizeof(float));
}

// dS after that, for the backward whose dQ reads the dK/dV kernel's dS
// (bf16, unsplit, 8-wave grids): per (b, h) S rounded up to 32 keys x ds_ld
// queries bf16 (S rounded up to 256), in 1 KiB blocks of 32 keys x 16
// queries.  0 where that path does not apply: f32, split calls, 4-wave grids
// (there the 4-wave dK/dV kernel's stores cost what dQ saves: c3 431 against
// 450 us), or a head's blocks spanning 4 GiB (the kernels' buffer offsets
// are 32-bit).
// Past FA_BWD_DS_MAX_BYTES of dS (16 GiB) a call keeps the recomputing path
// rather than ask for a workspace of that size.
int ds_ld_for(int32_t S) { return (S + 255) / 256 * 256; }
size_t bwd_ds_bytes(int32_t dtype, int32_t B, int32_t S, int32_t H) {
    if (dtype != FA_DTYPE_BF16 || split_for(dtype, B, S, H) > 1 || fa::attn_waves(B, H, S) != 8) return 0;
    const int64_t head = (int64_t)(S + 31) / 32 * 32 * ds_ld_for(S) * 2;
    if (head >= (int64_t(1) << 32)) return 0;
    const size_t bytes = round256((size_t)B * H * head);
    return bytes > (size_t)FA_BWD_DS_MAX_BYTES ? 0 : bytes;
}

size_t bwd_workspace(int32_t dtype, int32_t B, int32_t S, int32_t H, int32_t D) {
    return bwd_min_workspace(dtype, B, S, H, D) + bwd_ds_bytes(dtype, B, S, H);
}

// forward workspace of a split call: O partials [split][B,H,S][D] f32, then
// the partial LSEs [split][B,H,S] f32; 0 when the call does not split
size_t fwd_workspace(int32_t dtype, int32_t B, int32_t S, int32_t H, int32_t D) {
    const int split = split_for(dtype, B, S, H);
    if (split <= 1) return 0;
    return round256(fa::attn_split_elems(B, H, S, D, split) * sizeof(float)) +
           round256((size_t)split * B * H * S * sizeof(float));
}

#define FA_TRY(expr)                      \
    do {                                  \
        const fa_status st__ = (expr);    \
        if (st__ != FA_OK) return st__;   \
    } while (0)

}  // namespace

namespace fa {
hipError_t prepare_fwd_kernels();
hipError_t prepare_bwd_kernels();
hipError_t prepare_attn_kernels() {
    hipError_t e = prepare_fwd_kernels();
    if (e != hipSuccess) return e;
    return prepare_bwd_kernels();
}
}  // namespace fa

extern "C" {

int fa_version(void) { return FA_ABI_VERSION; }

const char *fa_last_error(void) { return g_err; }

const char *fa_op_name(void) { return "foundry-attn-bwd"; }

fa_status fa_init(int device) {
    FA_TRY(init_device(device));
    {
        std::lock_guard<std::mutex> lk(g_init_mu);
        FA_TRY(setup_scratch_locked(device));
    }
    return ok();
}

fa_status fa_attn_fwd(const fa_attn_fwd_args *a, void *stream) {
    if (!a) return fail(FA_ERR_INVALID_ARG, "args is NULL");
    FA_TRY(check_attn_shape(a->dtype, a->batch, a->seq, a->heads, a->head_dim, a->scale));
    FA_TRY(check_view("q", a->q, a->q_stride, a->dtype));
    FA_TRY(check_view("k", a->k, a->k_stride, a->dtype));
    FA_TRY(check_view("v", a->v, a->v_stride, a->dtype));
    FA_TRY(check_view("o", a->o, a->o_stride, a->dtype));
    if (!a->lse || !aligned(a->lse, 4)) return fail(FA_ERR_INVALID_ARG, "lse is NULL or misaligned");
    if (a->dtype == FA_DTYPE_BF16) {
        FA_TRY(check_buffer_view("k", a->k_stride, a->seq, a->head_dim));
        FA_TRY(check_buffer_view("v", a->v_stride, a->seq, a->head_dim));
    }
    FA_TRY(init_current());

    fa::AttnFwdParams p{};
    p.q = a->q; p.k = a->k; p.v = a->v; p.o = a->o; p.lse = a->lse; p.keep = a->key_keep;
    p.q_sb = a->q_stride.b; p.q_ss = a->q_stride.s; p.q_sh = a->q_stride.h;
    p.k_sb = a->k_stride.b; p.k_ss = a->k_stride.s; p.k_sh = a->k_stride.h;
    p.v_sb = a->v_stride.b; p.v_ss = a->v_stride.s; p.v_sh = a->v_stride.h;
    p.o_sb = a->o_stride.b; p.o_ss = a->o_stride.s; p.o_sh = a->o_stride.h;
    p.B = a->batch; p.S = a->seq; p.H = a->heads;
    p.scale = a->scale;
    p.scale_log2 = a->scale * 1.4426950408889634f;
    p.split = 1;
    if (a->workspace) {
        const size_t need = fwd_workspace(a->dtype, a->batch, a->seq, a->heads, a->head_dim);
        if (!aligned(a->workspace, 256)) return fail(FA_ERR_INVALID_ARG, "workspace is not 256-byte aligned");
        if (a->workspace_bytes < need)
            return fail(FA_ERR_INVALID_ARG,
                        "workspace of %zu bytes is smaller than the %zu a split forward needs (NULL runs unsplit)",
                        a->workspace_bytes, need);
        if (need > 0) {
            p.split = split_for(a->dtype, a->batch, a->seq, a->heads);
            p.part_o = static_cast<float *>(a->workspace);
            p.part_lse = reinterpret_cast<float *>(
                static_cast<char *>(a->workspace) +
                round256(fa::attn_split_elems(a->batch, a->heads, a->seq, a->head_dim, p.split) * sizeof(float)));
        }
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    const hipError_t e = a->dtype == FA_DTYPE_BF16 ? fa::launch_attn_fwd_bf16(p, a->head_dim, s)
                                                   : fa::launch_attn_fwd_f32(p, a->head_dim, s);
    if (e != hipSuccess) return hip_fail(e, "attention forward launch");
    return ok();
}

size_t fa_attn_fwd_workspace_size(const fa_attn_fwd_args *a) {
    if (!a || a->batch < 1 || a->seq < 1 || a->heads < 1 || (a->head_dim != 64 && a->head_dim != 128)) return 0;
    return fwd_workspace(a->dtype, a->batch, a->seq, a->heads, a->head_dim);
}

size_t fa_attn_bwd_workspace_size(const fa_attn_bwd_args *a) {
    if (!a || a->batch < 1 || a->seq < 1 || a->heads < 1 || (a->head_dim != 64 && a->head_dim != 128)) return 0;
    return bwd_workspace(a->dtype, a->batch, a->seq, a->heads, a->head_dim);
}

size_t fa_attn_bwd_min_workspace_size(const fa_attn_bwd_args *a) {
    if (!a || a->batch < 1 || a->seq < 1 || a->heads < 1 || (a->head_dim != 64 && a->head_dim != 128)) return 0;
    return bwd_min_workspace(a->dtype, a->batch, a->seq, a->heads, a->head_dim);
}

fa_status fa_attn_bwd(const fa_attn_bwd_args *a, void *stream) {
    return fa_attn_bwd_phase(a, FA_BWD_ALL, stream);
}

}  // extern "C"

namespace {
// With the 4-wave kernels (fa::attn_waves) the whole bf16 backward runs dQ beside
// dK/dV: the two kernels are independent after the pre-pass, and two
// 4-wave workgroups per CU let them fill the partial last wave each leaves
// on its own (measured 2.4% off a 4-wave c2 backward, results
// bit-identical).  The 8-wave kernels each fill a CU's registers alone, and
// there running them side by side measured 4% slower than in order, so they
// run in order on the caller's stream.  Per host thread and device: one side
// stream (default priority) and two events, made on first use and kept for
// the thread's life, so concurrent callers on other threads never share
// them.
struct BwdFork {
    hipStream_t side = nullptr;
    hipEvent_t pre = nullptr, done = nullptr;
};
constexpr int kMaxForkDevices = 64;
thread_local BwdFork g_fork[kMaxForkDevices];

hipError_t fork_for_current(BwdFork **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxForkDevices) return hipErrorInvalidDevice;
    BwdFork &f = g_fork[dev];
    if (!f.side) {
        hipStream_t st = nullptr;
        hipEvent_t e0 = nullptr, e1 = nullptr;
        // a partial failure releases what was made (the caller then runs the
        // backward in order on its own stream)
        if ((e = hipStreamCreateWithFlags(&st, hipStreamNonBlocking)) != hipSuccess) return e;
        if ((e = hipEventCreateWithFlags(&e0, hipEventDisableTiming)) != hipSuccess) {
            (void)hipStreamDestroy(st);
            return e;
        }
        if ((e = hipEventCreateWithFlags(&e1, hipEventDisableTiming)) != hipSuccess) {
            (void)hipEventDestroy(e0);
            (void)hipStreamDestroy(st);
            return e;
        }
        f.side = st;
        f.pre = e0;
        f.done = e1;
    }
    *out = &f;
    return hipSuccess;
}

// pre-pass and dK/dV on s; dQ on the side stream after the pre-pass; s then
// waits for dQ, so everything the caller queues on s afterwards sees all
// three results (and may reuse the workspace).
hipError_t launch_bwd_forked(const fa::AttnBwdParams &p, int D, hipStream_t s) {
    // through the stored dS, dQ follows dK/dV
    if (p.ds || fa::attn_waves(p.B, p.H, p.S) == 8) return fa::launch_attn_bwd_bf16(p, D, FA_BWD_ALL, s);
    BwdFork *f = nullptr;
    if (fork_for_current(&f) != hipSuccess) return fa::launch_attn_bwd_bf16(p, D, FA_BWD_ALL, s);
    hipError_t e = fa::launch_attn_bwd_bf16(p, D, FA_BWD_PREPASS, s);
    if (e == hipSuccess) e = hipEventRecord(f->pre, s);
    if (e == hipSuccess) e = fa::launch_attn_bwd_bf16(p, D, FA_BWD_DKDV, s);
    if (e == hipSuccess) e = hipStreamWaitEvent(f->side, f->pre, 0);
    if (e == hipSuccess) e = fa::launch_attn_bwd_bf16(p, D, FA_BWD_DQ, f->side);
    if (e == hipSuccess) e = hipEventRecord(f->done, f->side);
    if (e == hipSuccess) e = hipStreamWaitEvent(s, f->done, 0);
    return e;
}


// Validates a backward call's shapes, views and LSE (not its workspace).
fa_status check_bwd_args(const fa_attn_bwd_args *a) {
    FA_TRY(check_attn_shape(a->dtype, a->batch, a->seq, a->heads, a->head_dim, a->scale));
    FA_TRY(check_view("q", a->q, a->q_stride, a->dtype));
    FA_TRY(check_view("k", a->k, a->k_stride, a->dtype));
    FA_TRY(check_view("v", a->v, a->v_stride, a->dtype));
    FA_TRY(check_view("o", a->o, a->o_stride, a->dtype));
    FA_TRY(check_view("dout", a->dout, a->do_stride, a->dtype));
    FA_TRY(check_view("dq", a->dq, a->dq_stride, a->dtype));
    FA_TRY(check_view("dk", a->dk, a->dk_stride, a->dtype));
    FA_TRY(check_view("dv", a->dv, a->dv_stride, a->dtype));
    if (!a->lse || !aligned(a->lse, 4)) return fail(FA_ERR_INVALID_ARG, "lse is NULL or misaligned");
    if (a->dtype == FA_DTYPE_BF16) {
        FA_TRY(check_buffer_view("q", a->q_stride, a->seq, a->head_dim));
        FA_TRY(check_buffer_view("k", a->k_stride, a->seq, a->head_dim));
        FA_TRY(check_buffer_view("v", a->v_stride, a->seq, a->head_dim));
        FA_TRY(check_buffer_view("dout", a->do_stride, a->seq, a->head_dim));
    }
    return FA_OK;
}

// Kernel parameters of a validated backward call whose scratch starts at ws
// (delta rows, lse2 rows, then, for split > 1, the three partial arrays, and
// with ds the dS^T rows: the caller passed the full workspace).
void fill_bwd_params(const fa_attn_bwd_args *a, char *ws, int split, bool ds, fa::AttnBwdParams &p) {
    p = fa::AttnBwdParams{};
    const size_t rows = round256((size_t)a->batch * a->heads * a->seq * sizeof(float));
    p.q = a->q; p.k = a->k; p.v = a->v; p.o = a->o; p.dout = a->dout; p.lse = a->lse;
    p.keep = a->key_keep; p.dq = a->dq; p.dk = a->dk; p.dv = a->dv;
    p.delta = reinterpret_cast<float *>(ws);
    p.lse2 = reinterpret_cast<float *>(ws + rows);
    p.q_sb = a->q_stride.b; p.q_ss = a->q_stride.s; p.q_sh = a->q_stride.h;
    p.k_sb = a->k_stride.b; p.k_ss = a->k_stride.s; p.k_sh = a->k_stride.h;
    p.v_sb = a->v_stride.b; p.v_ss = a->v_stride.s; p.v_sh = a->v_stride.h;
    p.o_sb = a->o_stride.b; p.o_ss = a->o_stride.s; p.o_sh = a->o_stride.h;
    p.do_sb = a->do_stride.b; p.do_ss = a->do_stride.s; p.do_sh = a->do_stride.h;
    p.dq_sb = a->dq_stride.b; p.dq_ss = a->dq_stride.s; p.dq_sh = a->dq_stride.h;
    p.dk_sb = a->dk_stride.b; p.dk_ss = a->dk_stride.s; p.dk_sh = a->dk_stride.h;
    p.dv_sb = a->dv_stride.b; p.dv_ss = a->dv_stride.s; p.dv_sh = a->dv_stride.h;
    p.B = a->batch; p.S = a->seq; p.H = a->heads;
    p.scale = a->scale;
    p.scale_log2 = a->scale * 1.4426950408889634f;
    p.split = split;
    if (split > 1) {
        const size_t part = round256(
            fa::attn_split_elems(a->batch, a->heads, a->seq, a->head_dim, split) * sizeof(float));
        char *base = ws + 2 * rows;
        p.part_dq = reinterpret_cast<float *>(base);
        p.part_dk = reinterpret_cast<float *>(base + part);
        p.part_dv = reinterpret_cast<float *>(base + 2 * part);
    }
    if (ds) {
        p.ds = ws + bwd_min_workspace(a->dtype, a->batch, a->seq, a->heads, a->head_dim);
        p.ds_ld = ds_ld_for(a->seq);
    }
}
}  // namespace

extern "C" {

fa_status fa_attn_bwd_phase(const fa_attn_bwd_args *a, int32_t phase, void *stream) {
    if (!a) return fail(FA_ERR_INVALID_ARG, "args is NULL");
    if (phase < FA_BWD_ALL || phase > FA_BWD_DQ)
        return fail(FA_ERR_INVALID_ARG, "unknown backward phase %d", phase);
    FA_TRY(check_bwd_args(a));
    const size_t need = bwd_min_workspace(a->dtype, a->batch, a->seq, a->heads, a->head_dim);
    const size_t ds = bwd_ds_bytes(a->dtype, a->batch, a->seq, a->heads);
    if (!a->workspace || !aligned(a->workspace, 256))
        return fail(FA_ERR_INVALID_ARG, "workspace is NULL or not 256-byte aligned");
    if (a->workspace_bytes < need)
        return fail(FA_ERR_INVALID_ARG, "workspace of %zu bytes is smaller than the %zu needed",
                    a->workspace_bytes, need);
    FA_TRY(init_current());

    fa::AttnBwdParams p;
    fill_bwd_params(a, static_cast<char *>(a->workspace), split_for(a->dtype, a->batch, a->seq, a->heads),
                    ds > 0 && a->workspace_bytes >= need + ds, p);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const hipError_t e = a->dtype != FA_DTYPE_BF16 ? fa::launch_attn_bwd_f32(p, a->head_dim, phase, s)
                         : phase == FA_BWD_ALL     ? launch_bwd_forked(p, a->head_dim, s)
                                                   : fa::launch_attn_bwd_bf16(p, a->head_dim, phase, s);
    if (e != hipSuccess) return hip_fail(e, "attention backward launch");
    return ok();
}

fa_status fa_attn_bwd_noalloc(const fa_attn_bwd_args *a, void *stream) {
    if (!a) return fail(FA_ERR_INVALID_ARG, "args is NULL");
    FA_TRY(check_bwd_args(a));
    if (a->workspace || a->workspace_bytes)
        return fail(FA_ERR_INVALID_ARG,
                    "fa_attn_bwd_noalloc takes no workspace (workspace must be NULL, workspace_bytes 0)");
    const int64_t rows = (int64_t)a->batch * a->heads * a->seq;
    if (rows > FA_BWD_NOALLOC_MAX_ROWS)
        return fail(FA_ERR_INVALID_ARG,
                    "batch*heads*seq = %lld exceeds the %d rows the no-allocation scratch holds (%d bytes "
                    "per device); call fa_attn_bwd with a workspace",
                    (long long)rows, FA_BWD_NOALLOC_MAX_ROWS, kNoallocScratchBytes);
    FA_TRY(init_current());
    char *ws = nullptr;
    FA_TRY(scratch_for_current(&ws));

    // never split (the split partials would not fit), every launch in order on
    // the caller's stream (no side stream to create)
    fa::AttnBwdParams p;
    fill_bwd_params(a, ws, 1, false, p);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const hipError_t e = a->dtype != FA_DTYPE_BF16 ? fa::launch_attn_bwd_f32(p, a->head_dim, FA_BWD_ALL, s)
                                                   : fa::launch_attn_bwd_bf16(p, a->head_dim, FA_BWD_ALL, s);
    if (e != hipSuccess) return hip_fail(e, "attention backward launch");
    return ok();
}

}  // extern "C"

// The prologue kernels address a batch item's rows with 32-bit offsets made
// of 24-bit products: token and head strides below 2^24 elements, and the
// rows of one batch item within 2^31 elements of its first.
static fa_status check_prologue_span(const char *name, const fa_strides &st, int32_t tokens, int32_t heads,
                                     int32_t D) {
    if (st.s >= (int64_t(1) << 24) || st.h >= (int64_t(1) << 24))
        return fail(FA_ERR_UNSUPPORTED, "%s token/head strides (%lld, %lld) must be < 2^24 elements", name,
                    (long long)st.s, (long long)st.h);
    const int64_t span = (int64_t)(tokens - 1) * st.s + (int64_t)(heads - 1) * st.h + D;
    if (span >= (int64_t(1) << 31))
        return fail(FA_ERR_UNSUPPORTED, "%s spans %lld elements per batch item; this build addresses < 2^31", name,
                    (long long)span);
    return FA_OK;
}

static fa_status check_prologue(const fa_qk_prologue_args *a) {
    if (!a) return fail(FA_ERR_INVALID_ARG, "args is NULL");
    if (a->dtype != FA_DTYPE_BF16 && a->dtype != FA_DTYPE_F32)
        return fail(FA_ERR_INVALID_ARG, "unknown dtype %d", a->dtype);
    if (a->batch < 1 || a->tokens < 1 || a->heads < 1)
        return fail(FA_ERR_INVALID_ARG, "batch/tokens/heads must be >= 1");
    if ((int64_t)a->tokens * a->heads >= (int64_t(1) << 31) || a->batch > 65535)
        return fail(FA_ERR_UNSUPPORTED, "tokens * heads must be < 2^31 and batch <= 65535");
    // the kernels form a row's token and head with 24-bit products and an f32
    // quotient estimate that is exact for heads <= 1024
    if (a->tokens >= (1 << 24) || a->heads > 1024)
        return fail(FA_ERR_UNSUPPORTED, "tokens %d, heads %d: this build needs tokens < 2^24 and heads <= 1024",
                    a->tokens, a->heads);
    if (a->head_dim != 64 && a->head_dim != 128)
        return fail(FA_ERR_UNSUPPORTED, "head_dim %d: this build implements 64 and 128", a->head_dim);
    if (!(a->eps >= 0.f) || !isfinite(a->eps)) return fail(FA_ERR_INVALID_ARG, "eps must be finite, >= 0");
    if (a->n_axes < 1 || a->n_axes > FA_MAX_ROPE_AXES)
        return fail(FA_ERR_INVALID_ARG, "n_axes %d outside 1..%d", a->n_axes, FA_MAX_ROPE_AXES);
    int sum = 0;
    for (int i = 0; i < a->n_axes; ++i) {
        if (a->axes[i] <= 0 || (a->axes[i] & 1))
            return fail(FA_ERR_INVALID_ARG, "rope axis %d width %d must be even and > 0", i, a->axes[i]);
        sum += a->axes[i];
    }
    if (sum != a->head_dim)
        return fail(FA_ERR_INVALID_ARG, "rope axes sum to %d, head_dim is %d", sum, a->head_dim);
    if (a->y_seq_offset < 0) return fail(FA_ERR_INVALID_ARG, "y_seq_offset < 0");
    FA_TRY(check_view("x", a->x, a->x_stride, a->dtype));
    FA_TRY(check_view("y", a->y, a->y_stride, a->dtype));
    FA_TRY(check_prologue_span("x", a->x_stride, a->tokens, a->heads, a->head_dim));
    FA_TRY(check_prologue_span("y", a->y_stride, a->tokens, a->heads, a->head_dim));
    const size_t elt = a->dtype == FA_DTYPE_BF16 ? 2 : 4;
    if (!a->weight || !aligned(a->weight, elt)) return fail(FA_ERR_INVALID_ARG, "weight is NULL or misaligned");
    if (!a->cos || !a->sin || !aligned(a->cos, elt) || !aligned(a->sin, elt))
        return fail(FA_ERR_INVALID_ARG, "cos/sin table is NULL or misaligned");
    return FA_OK;
}

static void fill_prologue(const fa_qk_prologue_args *a, fa::QkPrologueParams &p) {
    p.x = a->x; p.x_sb = a->x_stride.b; p.x_ss = a->x_stride.s; p.x_sh = a->x_stride.h;
    p.w = a->weight; p.cos = a->cos; p.sin = a->sin;
    p.y = a->y; p.y_sb = a->y_stride.b; p.y_ss = a->y_stride.s; p.y_sh = a->y_stride.h;
    p.y_off = a->y_seq_offset;
    p.B = a->batch; p.T = a->tokens; p.H = a->heads; p.D = a->head_dim; p.eps = a->eps;
    p.n_axes = a->n_axes;
    for (int i = 0; i < FA_MAX_ROPE_AXES; ++i) p.axes[i] = i < a->n_axes ? a->axes[i] : 0;
}

// The bf16 rowdot (u = x·Aᵀ) addresses one workgroup's rows of x, up to 64,
// and the whole [r, K] factor with 32-bit buffer offsets.
static fa_status check_rowdot_span(const char *name, int64_t ld, int32_t rows, int32_t k, int32_t r) {
    const int64_t span = ((int64_t)(std::min(rows, 64) - 1) * ld + k) * 2;
    if (span >= (int64_t(1) << 32) || (int64_t)r * k * 2 >= (int64_t(1) << 32))
        return fail(FA_ERR_UNSUPPORTED, "%s: 64 rows of stride %lld, or the rank factor, span 4 GiB or more", name,
                    (long long)ld);
    return FA_OK;
}

static fa_status check_lora(const fa_lora_args *a) {
    if (!a) return fail(FA_ERR_INVALID_ARG, "args is NULL");
    if (a->dtype != FA_DTYPE_BF16 && a->dtype != FA_DTYPE_F32)
        return fail(FA_ERR_INVALID_ARG, "unknown dtype %d", a->dtype);
    if (a->tokens < 1 || a->in_features < 1 || a->out_features < 1)
        return fail(FA_ERR_INVALID_ARG, "tokens/in_features/out_features must be >= 1");
    if (a->rank < 1 || a->rank > 32)
        return fail(FA_ERR_UNSUPPORTED, "rank %d: this build implements 1..32", a->rank);
    if (!isfinite(a->scale)) return fail(FA_ERR_INVALID_ARG, "scale must be finite");
    const int kmul = a->dtype == FA_DTYPE_BF16 ? 16 : 2;
    if (a->in_features % kmul || a->out_features % kmul)
        return fail(FA_ERR_UNSUPPORTED, "in/out features must be multiples of %d", kmul);
    const size_t elt = a->dtype == FA_DTYPE_BF16 ? 2 : 4;
    if (!a->x || !aligned(a->x, 16) || a->ldx < a->in_features || (a->ldx * (int64_t)elt) % 16)
        return fail(FA_ERR_INVALID_ARG, "x is NULL, misaligned, or ldx < in_features");
    if (!a->a || !aligned(a->a, 16)) return fail(FA_ERR_INVALID_ARG, "a is NULL or misaligned");
    if (!a->b || !aligned(a->b, elt)) return fail(FA_ERR_INVALID_ARG, "b is NULL or misaligned");
    if (!a->u || !aligned(a->u, 4)) return fail(FA_ERR_INVALID_ARG, "u is NULL or misaligned");
    if (a->dtype == FA_DTYPE_BF16) FA_TRY(check_rowdot_span("x", a->ldx, a->tokens, a->in_features, a->rank));
    return FA_OK;
}

static void fill_lora(const fa_lora_args *a, fa::LoraParams &p) {
    p.x = a->x; p.ldx = a->ldx; p.a = a->a; p.b = a->b; p.u = a->u; p.y = a->y; p.ldy = a->ldy;
    p.N = a->tokens; p.K = a->in_features; p.M = a->out_features; p.r = a->rank; p.scale = a->scale;
}

namespace fa {
size_t lora_bwd_workspace_bytes(int N, int K, int M, int r, int elt);
}

extern "C" {

fa_status fa_qk_prologue_fwd(const fa_qk_prologue_args *a, void *stream) {
    return fa_qk_prologue_fwd_multi(a, 1, stream);
}

fa_status fa_qk_prologue_bwd(const fa_qk_prologue_bwd_args *a, void *stream) {
    return fa_qk_prologue_bwd_multi(a, 1, stream);
}

// Rows [off, off + T) of segments i and j overlap in one output view.
static bool rows_overlap(const void *yi, const fa_strides &si, int oi, int ti, const void *yj, const fa_strides &sj,
                         int oj, int tj) {
    if (yi != yj || si.b != sj.b || si.s != sj.s || si.h != sj.h) return false;
    return oi < oj + tj && oj < oi + ti;
}

static fa_status check_prologue_set(const fa_qk_prologue_args *const *segs, int32_t count) {
    if (count < 1 || count > FA_MAX_PROLOGUE_SEGS)
        return fail(FA_ERR_INVALID_ARG, "count %d outside 1..%d", count, FA_MAX_PROLOGUE_SEGS);
    for (int i = 1; i < count; ++i)
        if (segs[i]->dtype != segs[0]->dtype || segs[i]->head_dim != segs[0]->head_dim)
            return fail(FA_ERR_INVALID_ARG, "segment %d: dtype and head_dim must match segment 0", i);
    return FA_OK;
}

fa_status fa_qk_prologue_fwd_multi(const fa_qk_prologue_args *a, int32_t count, void *stream) {
    if (!a) return fail(FA_ERR_INVALID_ARG, "args is NULL");
    if (count < 1 || count > FA_MAX_PROLOGUE_SEGS)
        return fail(FA_ERR_INVALID_ARG, "count %d outside 1..%d", count, FA_MAX_PROLOGUE_SEGS);
    const fa_qk_prologue_args *segs[FA_MAX_PROLOGUE_SEGS];
    fa::QkPrologueParams ps[FA_MAX_PROLOGUE_SEGS]{};
    for (int i = 0; i < count; ++i) {
        FA_TRY(check_prologue(&a[i]));
        segs[i] = &a[i];
        fill_prologue(&a[i], ps[i]);
        for (int j = 0; j < i; ++j)
            if (rows_overlap(a[i].y, a[i].y_stride, a[i].y_seq_offset, a[i].tokens, a[j].y, a[j].y_stride,
                             a[j].y_seq_offset, a[j].tokens))
                return fail(FA_ERR_INVALID_ARG, "segments %d and %d write overlapping rows of y", j, i);
    }
    FA_TRY(check_prologue_set(segs, count));
    FA_TRY(init_current());
    const hipError_t e = fa::launch_qk_prologue_fwd(ps, count, a[0].dtype, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "qk prologue forward launch");
    return ok();
}

fa_status fa_qk_prologue_bwd_multi(const fa_qk_prologue_bwd_args *a, int32_t count, void *stream) {
    if (!a) return fail(FA_ERR_INVALID_ARG, "args is NULL");
    if (count < 1 || count > FA_MAX_PROLOGUE_SEGS)
        return fail(FA_ERR_INVALID_ARG, "count %d outside 1..%d", count, FA_MAX_PROLOGUE_SEGS);
    const fa_qk_prologue_args *segs[FA_MAX_PROLOGUE_SEGS];
    fa::QkPrologueParams ps[FA_MAX_PROLOGUE_SEGS]{};
    for (int i = 0; i < count; ++i) {
        FA_TRY(check_prologue(&a[i].fwd));
        FA_TRY(check_view("dy", a[i].dy, a[i].fwd.y_stride, a[i].fwd.dtype));
        FA_TRY(check_view("dx", a[i].dx, a[i].dx_stride, a[i].fwd.dtype));
        FA_TRY(check_prologue_span("dx", a[i].dx_stride, a[i].fwd.tokens, a[i].fwd.heads, a[i].fwd.head_dim));
        segs[i] = &a[i].fwd;
        fill_prologue(&a[i].fwd, ps[i]);
        ps[i].dy = a[i].dy;
        ps[i].dx = a[i].dx;
        ps[i].dx_sb = a[i].dx_stride.b;
        ps[i].dx_ss = a[i].dx_stride.s;
        ps[i].dx_sh = a[i].dx_stride.h;
        for (int j = 0; j < i; ++j)
            if (rows_overlap(a[i].dx, a[i].dx_stride, 0, a[i].fwd.tokens, a[j].dx, a[j].dx_stride, 0,
                             a[j].fwd.tokens))
                return fail(FA_ERR_INVALID_ARG, "segments %d and %d write the same dx rows", j, i);
    }
    FA_TRY(check_prologue_set(segs, count));
    FA_TRY(init_current());
    const hipError_t e = fa::launch_qk_prologue_bwd(ps, count, a[0].fwd.dtype, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "qk prologue backward launch");
    return ok();
}

static uint16_t to_bf16_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

fa_status fa_rope_tables_host(const float *positions, int32_t n_pos, int32_t n_axes,
                              const int32_t *axes, float theta, int32_t dtype, void *cos_out,
                              void *sin_out) {
    if (!positions || !axes || !cos_out || !sin_out) return fail(FA_ERR_INVALID_ARG, "NULL pointer");
    if (n_pos < 0 || n_axes < 1 || n_axes > FA_MAX_ROPE_AXES)
        return fail(FA_ERR_INVALID_ARG, "bad n_pos / n_axes");
    if (dtype != FA_DTYPE_BF16 && dtype != FA_DTYPE_F32)
        return fail(FA_ERR_INVALID_ARG, "unknown dtype %d", dtype);
    if (!isfinite(theta) || !(theta > 0.f)) return fail(FA_ERR_INVALID_ARG, "theta must be > 0");
    int D = 0;
    for (int a = 0; a < n_axes; ++a) {
        if (axes[a] <= 0 || (axes[a] & 1)) return fail(FA_ERR_INVALID_ARG, "axis widths must be even, > 0");
        D += axes[a];
    }
    for (int p = 0; p < n_pos; ++p) {
        int off = 0;
        for (int a = 0; a < n_axes; ++a) {
            const int w = axes[a], half = w / 2;
            for (int j = 0; j < half; ++j) {
                const float inv = powf(theta, -2.0f * (float)j / (float)w);
                const float f = positions[(int64_t)p * n_axes + a] * inv;
                const float c = cosf(f), s = sinf(f);
                for (int rep = 0; rep < 2; ++rep) {
                    const int64_t i = (int64_t)p * D + off + rep * half + j;
                    if (dtype == FA_DTYPE_F32) {
                        static_cast<float *>(cos_out)[i] = c;
                        static_cast<float *>(sin_out)[i] = s;
                    } else {
                        static_cast<uint16_t *>(cos_out)[i] = to_bf16_bits(c);
                        static_cast<uint16_t *>(sin_out)[i] = to_bf16_bits(s);
                    }
                }
            }
            off += w;
        }
    }
    return ok();
}

fa_status fa_lora_fwd(const fa_lora_args *a, void *stream) {
    FA_TRY(check_lora(a));
    const size_t elt = a->dtype == FA_DTYPE_BF16 ? 2 : 4;
    if (!a->y || !aligned(a->y, elt) || a->ldy < a->out_features)
        return fail(FA_ERR_INVALID_ARG, "y is NULL, misaligned, or ldy < out_features");
    FA_TRY(init_current());
    fa::LoraParams p{};
    fill_lora(a, p);
    const hipError_t e = fa::launch_lora_fwd(p, a->dtype, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "lora forward launch");
    return ok();
}

size_t fa_lora_bwd_workspace_size(const fa_lora_bwd_args *a) {
    if (!a || a->fwd.tokens < 1 || a->fwd.rank < 1 || a->fwd.in_features < 1 || a->fwd.out_features < 1)
        return 0;
    return fa::lora_bwd_workspace_bytes(a->fwd.tokens, a->fwd.in_features, a->fwd.out_features,
                                        a->fwd.rank, a->fwd.dtype == FA_DTYPE_BF16 ? 2 : 4);
}

fa_status fa_lora_bwd(const fa_lora_bwd_args *a, void *stream) {
    if (!a) return fail(FA_ERR_INVALID_ARG, "args is NULL");
    FA_TRY(check_lora(&a->fwd));
    const size_t elt = a->fwd.dtype == FA_DTYPE_BF16 ? 2 : 4;
    if (!a->dy || !aligned(a->dy, 16) || a->ldy < a->fwd.out_features || (a->ldy * (int64_t)elt) % 16)
        return fail(FA_ERR_INVALID_ARG, "dy is NULL, misaligned, or ldy < out_features");
    if (a->fwd.dtype == FA_DTYPE_BF16)
        FA_TRY(check_rowdot_span("dy", a->ldy, a->fwd.tokens, a->fwd.out_features, a->fwd.rank));
    if (!a->da || !a->db || !aligned(a->da, 4) || !aligned(a->db, 4))
        return fail(FA_ERR_INVALID_ARG, "da/db is NULL or misaligned");
    if (a->dx && (!aligned(a->dx, elt) || a->ldx < a->fwd.in_features))
        return fail(FA_ERR_INVALID_ARG, "dx misaligned or ldx < in_features");
    const size_t need = fa_lora_bwd_workspace_size(a);
    if (!a->workspace || !aligned(a->workspace, 256) || a->workspace_bytes < need)
        return fail(FA_ERR_INVALID_ARG, "workspace missing, misaligned or smaller than %zu bytes", need);
    FA_TRY(init_current());
    fa::LoraParams p{};
    fill_lora(&a->fwd, p);
    p.dy = a->dy; p.lddy = a->ldy; p.da = a->da; p.db = a->db; p.dx = a->dx; p.lddx = a->ldx;
    p.work = static_cast<float *>(a->workspace);
    const hipError_t e = fa::launch_lora_bwd(p, a->fwd.dtype, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "lora backward launch");
    return ok();
}

static fa_status check_lora_part(int32_t dtype, int32_t tokens, int32_t features, int32_t rank, float scale,
                                 const char *fname) {
    if (dtype != FA_DTYPE_BF16) return fail(FA_ERR_UNSUPPORTED, "adapter pieces are bf16 only");
    if (tokens < 1 || rank < 1 || rank > 64) return fail(FA_ERR_INVALID_ARG, "tokens >= 1 and rank 1..64");
    if (features < 16 || features % 16) return fail(FA_ERR_UNSUPPORTED, "%s must be a multiple of 16", fname);
    if (!isfinite(scale)) return fail(FA_ERR_INVALID_ARG, "scale must be finite");
    return FA_OK;
}

static fa_status check_rank_view(const char *name, const void *p, int64_t ld, int32_t rank) {
    if (!p || !aligned(p, 2)) return fail(FA_ERR_INVALID_ARG, "%s is NULL or misaligned", name);
    if (ld < rank) return fail(FA_ERR_INVALID_ARG, "%s: ld %lld < rank %d", name, (long long)ld, rank);
    return FA_OK;
}

fa_status fa_lora_down(const fa_lora_down_args *a, void *stream) {
    if (!a) return fail(FA_ERR_INVALID_ARG, "args is NULL");
    FA_TRY(check_lora_part(a->dtype, a->tokens, a->in_features, a->rank, a->scale, "in_features"));
    if (!a->x || !aligned(a->x, 16) || a->ldx < a->in_features || (a->ldx * 2) % 16)
        return fail(FA_ERR_INVALID_ARG, "x is NULL, misaligned, or ldx < in_features");
    if (!a->a || !aligned(a->a, 16)) return fail(FA_ERR_INVALID_ARG, "a is NULL or not 16-byte aligned");
    FA_TRY(check_rank_view("u", a->u, a->ldu, a->rank));
    FA_TRY(check_rowdot_span("x", a->ldx, a->tokens, a->in_features, a->rank));
    FA_TRY(init_current());
    const hipError_t e = fa::launch_lora_down_bf16(a->x, a->ldx, a->a, a->tokens, a->in_features, a->rank, a->scale,
                                                   a->u, a->ldu, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "lora down launch");
    return ok();
}

fa_status fa_lora_up(const fa_lora_up_args *a, void *stream) {
    if (!a) return fail(FA_ERR_INVALID_ARG, "args is NULL");
    FA_TRY(check_lora_part(a->dtype, a->tokens, a->out_features, a->rank, a->scale, "out_features"));
    FA_TRY(check_rank_view("u", a->u, a->ldu, a->rank));
    if (!a->b || !aligned(a->b, 2)) return fail(FA_ERR_INVALID_ARG, "b is NULL or misaligned");
    if (!a->y || !aligned(a->y, 2) || a->ldy < a->out_features)
        return fail(FA_ERR_INVALID_ARG, "y is NULL, misaligned, or ldy < out_features");
    FA_TRY(init_current());
    const hipError_t e = fa::launch_lora_up_bf16(a->u, a->ldu, a->b, a->tokens, a->out_features, a->rank, a->scale,
                                                 a->y, a->ldy, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "lora up launch");
    return ok();
}

static fa::LoraGradItem grad_item(const fa_lora_grad_args *a) {
    fa::LoraGradItem it{};
    it.u = a->u;
    it.ldu = a->ldu;
    it.x = a->x;
    it.ldx = a->ldx;
    it.N = a->tokens;
    it.C = a->features;
    it.R = a->rank;
    it.scale = a->scale;
    it.grad = a->grad;
    it.transpose = a->transpose != 0;
    return it;
}

static fa_status check_lora_grad(const fa_lora_grad_args *a) {
    if (!a) return fail(FA_ERR_INVALID_ARG, "args is NULL");
    FA_TRY(check_lora_part(a->dtype, a->tokens, a->features, a->rank, a->scale, "features"));
    FA_TRY(check_rank_view("u", a->u, a->ldu, a->rank));
    if (!a->x || !aligned(a->x, 16) || a->ldx < a->features || (a->ldx * 2) % 16)
        return fail(FA_ERR_INVALID_ARG, "x is NULL, misaligned, or ldx < features");
    if (!a->grad || !aligned(a->grad, 4)) return fail(FA_ERR_INVALID_ARG, "grad is NULL or misaligned");
    // the kernel reads u and x through buffer descriptors with 32-bit ranges
    const int64_t xspan = ((int64_t)(a->tokens - 1) * a->ldx + a->features) * 2;
    const int64_t uspan = ((int64_t)(a->tokens - 1) * a->ldu + a->rank) * 2 + 2;
    if (xspan >= (int64_t(1) << 32) || uspan >= (int64_t(1) << 32))
        return fail(FA_ERR_UNSUPPORTED, "u or x spans 4 GiB or more; this build addresses less per operand");
    return FA_OK;
}

size_t fa_lora_grad_workspace_size(const fa_lora_grad_args *a) {
    if (!a || a->tokens < 1 || a->features < 1 || a->rank < 1 || a->rank > 64) return 0;
    const fa::LoraGradItem it = grad_item(a);
    return fa::lora_grad_many_workspace_bytes(&it, 1);
}

fa_status fa_lora_grad(const fa_lora_grad_args *a, void *stream) {
    FA_TRY(check_lora_grad(a));
    const fa::LoraGradItem it = grad_item(a);
    const size_t need = fa::lora_grad_many_workspace_bytes(&it, 1);
    if (!a->workspace || !aligned(a->workspace, 256) || a->workspace_bytes < need)
        return fail(FA_ERR_INVALID_ARG, "workspace is NULL, not 256-byte aligned, or smaller than %zu bytes", need);
    FA_TRY(init_current());
    const hipError_t e = fa::launch_lora_grad_many_bf16(&it, 1, a->workspace, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "lora grad launch");
    return ok();
}

static constexpr int32_t kGradManyMax = 64;

size_t fa_lora_grad_many_workspace_size(const fa_lora_grad_args *args, int32_t count) {
    if (!args || count < 1 || count > kGradManyMax) return 0;
    fa::LoraGradItem items[kGradManyMax];
    for (int32_t i = 0; i < count; ++i) {
        const fa_lora_grad_args &a = args[i];
        if (a.tokens < 1 || a.features < 1 || a.rank < 1 || a.rank > 64) return 0;
        items[i] = grad_item(&a);
    }
    return fa::lora_grad_many_workspace_bytes(items, count);
}

fa_status fa_lora_grad_many(const fa_lora_grad_args *args, int32_t count, void *workspace, size_t workspace_bytes,
                            void *stream) {
    if (!args || count < 1 || count > kGradManyMax)
        return fail(FA_ERR_INVALID_ARG, "args is NULL or count not in 1..%d", kGradManyMax);
    fa::LoraGradItem items[kGradManyMax];
    for (int32_t i = 0; i < count; ++i) {
        FA_TRY(check_lora_grad(&args[i]));
        items[i] = grad_item(&args[i]);
    }
    const size_t need = fa::lora_grad_many_workspace_bytes(items, count);
    if (!workspace || !aligned(workspace, 256) || workspace_bytes < need)
        return fail(FA_ERR_INVALID_ARG, "workspace is NULL, not 256-byte aligned, or smaller than %zu bytes", need);
    FA_TRY(init_current());
    const hipError_t e = fa::launch_lora_grad_many_bf16(items, count, workspace, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "lora grad launch");
    return ok();
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Block ops (include/foundry_block.h)
// ---------------------------------------------------------------------------
namespace {

size_t dtype_bytes(int32_t dt) { return dt == FA_DTYPE_BF16 ? 2 : 4; }

fa_status check_row_view(const char *name, const void *p, int64_t ld, int32_t cols, int32_t dtype) {
    if (!p) return fail(FA_ERR_INVALID_ARG, "%s is NULL", name);
    if (!aligned(p, 16)) return fail(FA_ERR_INVALID_ARG, "%s is not 16-byte aligned", name);
    if (ld < cols || (ld * (int64_t)dtype_bytes(dtype)) % 16)
        return fail(FA_ERR_INVALID_ARG, "%s: ld %lld must be >= cols %d and keep rows 16-byte aligned", name,
                    (long long)ld, cols);
    return FA_OK;
}
fa_status check_vec(const char *name, const void *p) {
    if (!p || !aligned(p, 16)) return fail(FA_ERR_INVALID_ARG, "%s is NULL or not 16-byte aligned", name);
    return FA_OK;
}
fa_status check_rows_shape(int32_t dtype, int32_t rows, int32_t cols, int32_t max_cols) {
    if (dtype != FA_DTYPE_BF16 && dtype != FA_DTYPE_F32) return fail(FA_ERR_INVALID_ARG, "unknown dtype %d", dtype);
    if (rows < 1 || cols < 8 || cols % 8 || cols > max_cols)
        return fail(FA_ERR_INVALID_ARG, "rows %d / cols %d: need rows >= 1, 8 <= cols <= %d, cols %% 8 == 0", rows,
                    cols, max_cols);
    return FA_OK;
}

fa_status rows_op(const fa_rows_args *a, int op, void *stream) {
    if (!a) return fail(FA_ERR_INVALID_ARG, "args is NULL");
    FA_TRY(check_rows_shape(a->dtype, a->rows, a->cols, 1 << 30));
    FA_TRY(check_row_view("b", a->b, a->ldb, a->cols, a->dtype));
    FA_TRY(check_row_view("y", a->y, a->ldy, a->cols, a->dtype));
    if (op == 0) FA_TRY(check_vec("g", a->g));
    if (op == 2 || (op == 0 && a->x)) FA_TRY(check_row_view("x", a->x, a->ldx, a->cols, a->dtype));
    FA_TRY(init_current());
    fa::EltParams p{};
    p.x = (op == 0 || op == 2) ? a->x : nullptr;
    p.ldx = a->ldx;
    p.g = a->g;
    p.b = a->b;
    p.ldb = a->ldb;
    p.y = a->y;
    p.ldy = a->ldy;
    p.N = a->rows;
    p.C = a->cols;
    const hipError_t e = fa::launch_elementwise(p, op, a->dtype, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "elementwise launch");
    return ok();
}

fa_status check_ln(const fa_ln_mod_args *a) {
    FA_TRY(check_rows_shape(a->dtype, a->rows, a->cols, 4096));
    if (!(a->eps > 0.f) || !isfinite(a->eps)) return fail(FA_ERR_INVALID_ARG, "eps must be finite and > 0");
    FA_TRY(check_row_view("x", a->x, a->ldx, a->cols, a->dtype));
    FA_TRY(check_vec("shift", a->shift));
    FA_TRY(check_vec("scale", a->scale));
    return FA_OK;
}

fa::LnModParams ln_params(const fa_ln_mod_args *a) {
    fa::LnModParams p{};
    p.x = a->x;
    p.ldx = a->ldx;
    p.shift = a->shift;
    p.scale = a->scale;
    p.y = a->y;
    p.ldy = a->ldy;
    p.mean = a->mean;
    p.rstd = a->rstd;
    p.N = a->rows;
    p.C = a->cols;
    p.eps = a->eps;
    return p;
}

}  // namespace

extern "C" {

fa_status fa_ln_mod_fwd(const fa_ln_mod_args *a, void *stream) {
    if (!a) return fail(FA_ERR_INVALID_ARG, "args is NULL");
    FA_TRY(check_ln(a));
    FA_TRY(check_row_view("y", a->y, a->ldy, a->cols, a->dtype));
    if ((a->mean == nullptr) != (a->rstd == nullptr))
        return fail(FA_ERR_INVALID_ARG, "mean and rstd must both be given or both NULL");
    if (a->mean && (!aligned(a->mean, 4) || !aligned(a->rstd, 4)))
        return fail(FA_ERR_INVALID_ARG, "mean/rstd misaligned");
    FA_TRY(init_current());
    const hipError_t e = fa::launch_ln_mod_fwd(ln_params(a), a->dtype, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "layer-norm-mod launch");
    return ok();
}

fa_status fa_ln_mod_bwd(const fa_ln_mod_bwd_args *a, void *stream) {
    if (!a) return fail(FA_ERR_INVALID_ARG, "args is NULL");
    FA_TRY(check_ln(&a->fwd));
    if (!a->fwd.mean || !a->fwd.rstd || !aligned(a->fwd.mean, 4) || !aligned(a->fwd.rstd, 4))
        return fail(FA_ERR_INVALID_ARG, "mean and rstd (from the forward) are required");
    FA_TRY(check_row_view("dy", a->dy, a->lddy, a->fwd.cols, a->fwd.dtype));
    FA_TRY(check_row_view("dx", a->dx, a->lddx, a->fwd.cols, a->fwd.dtype));
    if (a->dres) FA_TRY(check_row_view("dres", a->dres, a->ldres, a->fwd.cols, a->fwd.dtype));
    FA_TRY(init_current());
    fa::LnModParams p = ln_params(&a->fwd);
    p.dy = a->dy;
    p.lddy = a->lddy;
    p.dres = a->dres;
    p.ldres = a->ldres;
    p.dx = a->dx;
    p.lddx = a->lddx;
    const hipError_t e = fa::launch_ln_mod_bwd(p, a->fwd.dtype, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "layer-norm-mod backward launch");
    return ok();
}

fa_status fa_gated_ln_mod_fwd(const fa_gated_ln_mod_args *a, void *stream) {
    if (!a) return fail(FA_ERR_INVALID_ARG, "args is NULL");
    const fa_ln_mod_args *l = &a->ln;
    FA_TRY(check_ln(l));
    FA_TRY(check_row_view("y", l->y, l->ldy, l->cols, l->dtype));
    if ((l->mean == nullptr) != (l->rstd == nullptr))
        return fail(FA_ERR_INVALID_ARG, "mean and rstd must both be given or both NULL");
    if (l->mean && (!aligned(l->mean, 4) || !aligned(l->rstd, 4)))
        return fail(FA_ERR_INVALID_ARG, "mean/rstd misaligned");
    FA_TRY(check_vec("g", a->g));
    FA_TRY(check_row_view("b", a->b, a->ldb, l->cols, l->dtype));
    FA_TRY(check_row_view("sum", a->sum, a->ldsum, l->cols, l->dtype));
    if (a->sum2) FA_TRY(check_row_view("sum2", a->sum2, a->ldsum2, l->cols, l->dtype));
    FA_TRY(init_current());
    fa::LnModParams p = ln_params(l);
    p.g = a->g;
    p.b = a->b;
    p.ldb = a->ldb;
    p.sum = a->sum;
    p.ldsum = a->ldsum;
    p.sum2 = a->sum2;
    p.ldsum2 = a->ldsum2;
    const hipError_t e = fa::launch_ln_mod_fwd(p, l->dtype, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "gated layer-norm-mod launch");
    return ok();
}

fa_status fa_ln_mod_bwd_gate(const fa_ln_mod_bwd_gate_args *a, void *stream) {
    if (!a) return fail(FA_ERR_INVALID_ARG, "args is NULL");
    const fa_ln_mod_bwd_args *w = &a->bwd;
    FA_TRY(check_ln(&w->fwd));
    if (!w->fwd.mean || !w->fwd.rstd || !aligned(w->fwd.mean, 4) || !aligned(w->fwd.rstd, 4))
        return fail(FA_ERR_INVALID_ARG, "mean and rstd (from the forward) are required");
    FA_TRY(check_row_view("dy", w->dy, w->lddy, w->fwd.cols, w->fwd.dtype));
    FA_TRY(check_row_view("dx", w->dx, w->lddx, w->fwd.cols, w->fwd.dtype));
    if (w->dres) FA_TRY(check_row_view("dres", w->dres, w->ldres, w->fwd.cols, w->fwd.dtype));
    FA_TRY(check_vec("g", a->g));
    FA_TRY(check_row_view("gdx", a->gdx, a->ldgdx, w->fwd.cols, w->fwd.dtype));
    FA_TRY(init_current());
    fa::LnModParams p = ln_params(&w->fwd);
    p.dy = w->dy;
    p.lddy = w->lddy;
    p.dres = w->dres;
    p.ldres = w->ldres;
    p.dx = w->dx;
    p.lddx = w->lddx;
    p.g = a->g;
    p.gdx = a->gdx;
    p.ldgdx = a->ldgdx;
    const hipError_t e = fa::launch_ln_mod_bwd(p, w->fwd.dtype, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "layer-norm-mod backward launch");
    return ok();
}

fa_status fa_gemm_bf16(const fa_gemm_args *a, void *stream) {
    if (!a) return fail(FA_ERR_INVALID_ARG, "args is NULL");
    if (a->epilogue < FA_GEMM_PLAIN || a->epilogue > FA_GEMM_DGELU)
        return fail(FA_ERR_INVALID_ARG, "unknown epilogue %d", a->epilogue);
    if (a->m < 256 || a->n < 256 || a->k < 64 || a->m % 256 || a->n % 256 || a->k % 64)
        return fail(FA_ERR_UNSUPPORTED, "m %d, n %d, k %d: this build needs m, n multiples of 256 and k of 64",
                    a->m, a->n, a->k);
    FA_TRY(check_row_view("a", a->a, a->lda, a->k, FA_DTYPE_BF16));
    FA_TRY(check_row_view("b", a->b, a->ldb, a->k, FA_DTYPE_BF16));
    FA_TRY(check_row_view("c", a->c, a->ldc, a->n, FA_DTYPE_BF16));
    if (a->epilogue == FA_GEMM_GELU) FA_TRY(check_row_view("c2", a->c2, a->ldc2, a->n, FA_DTYPE_BF16));
    if (a->epilogue == FA_GEMM_DGELU) FA_TRY(check_row_view("aux", a->aux, a->ldaux, a->n, FA_DTYPE_BF16));
    // buffer offsets within one 256-row block of a or b are 32-bit
    if ((255 * a->lda + a->k) * 2 >= (int64_t(1) << 31) || (255 * a->ldb + a->k) * 2 >= (int64_t(1) << 31))
        return fail(FA_ERR_UNSUPPORTED, "a 256-row block of a or b spans 2^31 bytes or more");
    FA_TRY(init_current());
    fa::GemmParams p{};
    p.a = a->a; p.lda = a->lda; p.b = a->b; p.ldb = a->ldb;
    p.c = a->c; p.ldc = a->ldc; p.c2 = a->c2; p.ldc2 = a->ldc2; p.aux = a->aux; p.ldaux = a->ldaux;
    p.M = a->m; p.N = a->n; p.K = a->k; p.epi = a->epilogue;
    const hipError_t e = fa::launch_gemm_tn_bf16(p, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "gemm launch");
    return ok();
}

fa_status fa_gated_residual(const fa_rows_args *a, void *stream) { return rows_op(a, 0, stream); }
fa_status fa_gelu_fwd(const fa_rows_args *a, void *stream) { return rows_op(a, 1, stream); }
fa_status fa_gelu_bwd(const fa_rows_args *a, void *stream) { return rows_op(a, 2, stream); }
fa_status fa_silu(const fa_rows_args *a, void *stream) { return rows_op(a, 3, stream); }

static fa_status check_swiglu(const fa_swiglu_args *a) {
    FA_TRY(check_rows_shape(a->dtype, a->rows, a->cols, 1 << 30));
    FA_TRY(check_row_view("gate", a->gate, a->ldgate, a->cols, a->dtype));
    FA_TRY(check_row_view("up", a->up, a->ldup, a->cols, a->dtype));
    return FA_OK;
}

fa_status fa_swiglu_fwd(const fa_swiglu_args *a, void *stream) {
    if (!a) return fail(FA_ERR_INVALID_ARG, "args is NULL");
    FA_TRY(check_swiglu(a));
    FA_TRY(check_row_view("y", a->y, a->ldy, a->cols, a->dtype));
    FA_TRY(init_current());
    fa::SwigluParams p{};
    p.gate = a->gate;
    p.ldg = a->ldgate;
    p.up = a->up;
    p.ldu = a->ldup;
    p.y = a->y;
    p.ldy = a->ldy;
    p.N = a->rows;
    p.C = a->cols;
    const hipError_t e = fa::launch_swiglu(p, false, a->dtype, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "swiglu launch");
    return ok();
}

fa_status fa_swiglu_bwd(const fa_swiglu_bwd_args *a, void *stream) {
    if (!a) return fail(FA_ERR_INVALID_ARG, "args is NULL");
    FA_TRY(check_swiglu(&a->fwd));
    FA_TRY(check_row_view("dy", a->dy, a->lddy, a->fwd.cols, a->fwd.dtype));
    FA_TRY(check_row_view("dgate", a->dgate, a->lddgate, a->fwd.cols, a->fwd.dtype));
    FA_TRY(check_row_view("dup", a->dup, a->lddup, a->fwd.cols, a->fwd.dtype));
    FA_TRY(init_current());
    fa::SwigluParams p{};
    p.gate = a->fwd.gate;
    p.ldg = a->fwd.ldgate;
    p.up = a->fwd.up;
    p.ldu = a->fwd.ldup;
    p.dy = a->dy;
    p.lddy = a->lddy;
    p.y = a->dgate;
    p.ldy = a->lddgate;
    p.dup = a->dup;
    p.lddup = a->lddup;
    p.N = a->fwd.rows;
    p.C = a->fwd.cols;
    const hipError_t e = fa::launch_swiglu(p, true, a->fwd.dtype, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "swiglu backward launch");
    return ok();
}

}  // extern "C"

namespace {
fa_status check_adamw(const fa_adamw_args *a) {
    if (!a) return fail(FA_ERR_INVALID_ARG, "args is NULL");
    if (a->dtype != FA_DTYPE_BF16 && a->dtype != FA_DTYPE_F32)
        return fail(FA_ERR_INVALID_ARG, "unknown dtype %d", a->dtype);
    if (a->n < 1) return fail(FA_ERR_INVALID_ARG, "n must be >= 1");
    if (a->step < 1) return fail(FA_ERR_INVALID_ARG, "step must be >= 1");
    if (!a->param || !a->grad || !a->m || !a->v || !aligned(a->param, dtype_bytes(a->dtype)) ||
        !aligned(a->grad, 4) || !aligned(a->m, 4) || !aligned(a->v, 4))
        return fail(FA_ERR_INVALID_ARG, "param/grad/m/v is NULL or misaligned");
    if (!(a->lr >= 0.0) || !(a->beta1 >= 0.0 && a->beta1 < 1.0) || !(a->beta2 >= 0.0 && a->beta2 < 1.0) ||
        !(a->eps > 0.0))
        return fail(FA_ERR_INVALID_ARG, "need lr >= 0, 0 <= beta < 1, eps > 0");
    return FA_OK;
}

// The step's f32 scalars, formed as the reference does (1 - beta and the
// bias corrections in f64, then rounded).
template <typename P>
void adamw_scalars(const fa_adamw_args *a, P &p) {
    const double b1 = a->beta1, b2 = a->beta2;
    p.lr = (float)a->lr;
    p.b1 = (float)b1;
    p.b2 = (float)b2;
    p.one_m_b1 = (float)(1.0 - b1);
    p.one_m_b2 = (float)(1.0 - b2);
    p.eps = (float)a->eps;
    p.ibc1 = (float)(1.0 / (1.0 - pow(b1, a->step)));
    p.ibc2 = (float)(1.0 / (1.0 - pow(b2, a->step)));
}
}  // namespace

extern "C" {

fa_status fa_adamw_step(const fa_adamw_args *a, void *stream) {
    FA_TRY(check_adamw(a));
    FA_TRY(init_current());
    fa::AdamwParams p{};
    p.param = a->param;
    p.grad = a->grad;
    p.m = a->m;
    p.v = a->v;
    p.n = a->n;
    adamw_scalars(a, p);
    const hipError_t e = fa::launch_adamw(p, a->dtype, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "adamw launch");
    return ok();
}

fa_status fa_copy2d_many(const fa_copy2d_args *args, int32_t count, void *stream) {
    if (!args || count < 1) return fail(FA_ERR_INVALID_ARG, "args is NULL or count < 1");
    for (int32_t i = 0; i < count; ++i) {
        const fa_copy2d_args &a = args[i];
        if (a.dtype != FA_DTYPE_BF16 && a.dtype != FA_DTYPE_F32)
            return fail(FA_ERR_INVALID_ARG, "view %d: unknown dtype %d", i, a.dtype);
        if (a.dtype != args[0].dtype) return fail(FA_ERR_INVALID_ARG, "view %d: dtype differs from view 0's", i);
        if (a.rows < 1 || a.cols < 1) return fail(FA_ERR_INVALID_ARG, "view %d: rows and cols must be >= 1", i);
        if (a.src_rs < 0 || a.src_cs < 0 || a.dst_rs < 0 || a.dst_cs < 0)
            return fail(FA_ERR_INVALID_ARG, "view %d: strides must be >= 0", i);
        const size_t eb = dtype_bytes(a.dtype);
        if (!a.src || !a.dst || !aligned(a.src, eb) || !aligned(a.dst, eb))
            return fail(FA_ERR_INVALID_ARG, "view %d: src or dst is NULL or misaligned", i);
    }
    FA_TRY(init_current());
    for (int32_t k0 = 0; k0 < count; k0 += fa::kCopyMany) {
        fa::Copy2dMany p{};
        p.count = count - k0 < fa::kCopyMany ? count - k0 : fa::kCopyMany;
        for (int k = 0; k < p.count; ++k) {
            const fa_copy2d_args &a = args[k0 + k];
            p.src[k] = a.src;
            p.dst[k] = a.dst;
            p.src_rs[k] = a.src_rs;
            p.src_cs[k] = a.src_cs;
            p.dst_rs[k] = a.dst_rs;
            p.dst_cs[k] = a.dst_cs;
            p.rows[k] = a.rows;
            p.cols[k] = a.cols;
        }
        const hipError_t e = fa::launch_copy2d_many(p, (int)dtype_bytes(args[0].dtype),
                                                    static_cast<hipStream_t>(stream));
        if (e != hipSuccess) return hip_fail(e, "copy launch");
    }
    return ok();
}

fa_status fa_adamw_step_many(const fa_adamw_args *args, int32_t count, void *stream) {
    if (!args || count < 1) return fail(FA_ERR_INVALID_ARG, "args is NULL or count < 1");
    for (int32_t i = 0; i < count; ++i) {
        FA_TRY(check_adamw(&args[i]));
        const fa_adamw_args &a = args[i], &z = args[0];
        if (a.dtype != z.dtype || a.lr != z.lr || a.beta1 != z.beta1 || a.beta2 != z.beta2 || a.eps != z.eps ||
            a.step != z.step)
            return fail(FA_ERR_INVALID_ARG, "tensor %d: dtype, lr, betas, eps and step must match tensor 0", i);
    }
    FA_TRY(init_current());
    for (int32_t k0 = 0; k0 < count; k0 += fa::kAdamwMany) {
        fa::AdamwMany p{};
        p.count = count - k0 < fa::kAdamwMany ? count - k0 : fa::kAdamwMany;
        for (int k = 0; k < p.count; ++k) {
            const fa_adamw_args &a = args[k0 + k];
            p.param[k] = a.param;
            p.grad[k] = a.grad;
            p.m[k] = a.m;
            p.v[k] = a.v;
            p.n[k] = a.n;
        }
        adamw_scalars(&args[0], p);
        const hipError_t e = fa::launch_adamw_many(p, args[0].dtype, static_cast<hipStream_t>(stream));
        if (e != hipSuccess) return hip_fail(e, "adamw launch");
    }
    return ok();
}

}  // extern "C"
