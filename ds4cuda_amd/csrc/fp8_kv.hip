// fp8_kv.hip — FP8 E4M3FN KV quantizer for gfx950.
//
// One 64-lane wave quantizes one 512-dim row: lane t owns dims [8t, 8t+8),
// so a 64-element scale block is 8 adjacent lanes and its max |x| is three
// DPP-class xor shuffles. The encoder is the exact bit-level
// round-to-nearest-even of ds4hip_common.h, not a table search. Loads and
// stores are 32 B / 16 B / 8 B per lane and fully coalesced per row.
//
// Two entry points:
//   * round trip (reference launcher, cuda/fp8_kv.cuh:62): fp32 in, fake-quant
//     fp32 out, tail copied through;
//   * append: writes the cache layout used by the decode kernels —
//     codes u8 [row][n_nope], scale exponents i8 [row][8] (7 used + 1 zero pad),
//     tail f16 [row][n_rot] — at caller-chosen physical rows.

#include "ds4hip_common.h"
#include "step_bodies.h"
#include "../../include/ds4hip.h"

using namespace ds4hip;

namespace {

constexpr int kRowsPerBlock = 4;   // 256 threads, 64 lanes per 512-dim row

// head_dim = 8 * lanes_per_row; lanes_per_row <= 64 and a multiple of 8.
template <bool kRoundTrip>
__global__ __launch_bounds__(256) void fp8_rows_kernel(
        const float *__restrict__ kv_in, float *__restrict__ kv_out,
        uint8_t *__restrict__ codes, int8_t *__restrict__ sexp, uint16_t *__restrict__ tail,
        int n_rows, int head_dim, int n_rot, long long row0,
        const long long *__restrict__ dst_rows) {
    const int lanes_per_row = head_dim >> 3;
    const int rows_per_block = 256 / 64;
    const int sub = threadIdx.x >> 6;              // row slot in the block
    const int t = threadIdx.x & 63;                // lane within the row
    const int row = blockIdx.x * rows_per_block + sub;
    if (row >= n_rows || t >= lanes_per_row) return;
    const long long prow = dst_rows ? dst_rows[row] : row0 + row;
    fp8_row_body<kRoundTrip>(kv_in, kv_out, codes, sexp, tail, row, head_dim, n_rot, prow, t);
}

// Three jobs over consecutive workgroup ranges, four rows (waves) each: the
// two FP8 row sets, then the fp32 row scatter.
struct RowsPushArgs {
    ds4hip_rows_push p;
    uint8_t *codes;
    int8_t *sexp;
    uint16_t *tail;
    int head_dim, n_rot;
    int blk[3];   // first workgroup of jobs 1 and 2, and the grid
};
__global__ __launch_bounds__(256) void rows_push_kernel(const RowsPushArgs A) {
    const int b = blockIdx.x, sub = threadIdx.x >> 6, t = threadIdx.x & 63;
    if (b < A.blk[1]) {
        const int k = b < A.blk[0] ? 0 : 1;
        const int row = (b - (k ? A.blk[0] : 0)) * 4 + sub;
        if (row >= A.p.fp8_n[k] || t >= (A.head_dim >> 3)) return;
        fp8_row_body<false>(A.p.fp8_src[k], nullptr, A.codes, A.sexp, A.tail, row, A.head_dim, A.n_rot,
                            A.p.fp8_dst[k][row], t);
        return;
    }
    const int row = (b - A.blk[1]) * 4 + sub;
    if (row < A.p.f32_n) row_copy_body(A.p.f32_src, row, A.p.f32_width, A.p.f32_dst, A.p.f32_dst_rows, t);
}

bool shape_ok(int head_dim, int n_rot) {
    return head_dim > 0 && head_dim <= 512 && head_dim % 64 == 0 && n_rot >= 0 &&
           n_rot % 8 == 0 && n_rot < head_dim && (head_dim - n_rot) % 64 == 0 &&
           (head_dim - n_rot) / 64 <= 8;
}

}  // namespace

extern "C" int ds4hip_fp8_kv_quantize_round_trip_f32(const float *kv_in, float *kv_out,
                                                     int n_rows, int head_dim, int n_rot,
                                                     void *stream) {
    if (n_rows < 0 || !shape_ok(head_dim, n_rot) || (n_rows > 0 && (!kv_in || !kv_out)))
        return ds4hip_set_last_error(kEINVAL);
    if (n_rows == 0) return 0;
    const int grid = (n_rows + kRowsPerBlock - 1) / kRowsPerBlock;
    hipLaunchKernelGGL(fp8_rows_kernel<true>, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                       kv_in, kv_out, nullptr, nullptr, nullptr, n_rows, head_dim, n_rot, 0LL,
                       nullptr);
    return ds4hip_set_last_error(hip_status(hipGetLastError()));
}

extern "C" int ds4hip_fp8_kv_quantize_append(const float *kv_in, int n_rows, int head_dim,
                                             int n_rot, uint8_t *codes, int8_t *sexp,
                                             uint16_t *tail, long long row0,
                                             const long long *dst_rows, void *stream) {
    if (n_rows < 0 || !shape_ok(head_dim, n_rot) || row0 < 0 ||
        (n_rows > 0 && (!kv_in || !codes || !sexp || (n_rot > 0 && !tail))))
        return ds4hip_set_last_error(kEINVAL);
    if (n_rows == 0) return 0;
    const int grid = (n_rows + kRowsPerBlock - 1) / kRowsPerBlock;
    hipLaunchKernelGGL(fp8_rows_kernel<false>, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                       kv_in, nullptr, codes, sexp, tail, n_rows, head_dim, n_rot, row0,
                       dst_rows);
    return ds4hip_set_last_error(hip_status(hipGetLastError()));
}

extern "C" int ds4hip_batch_rows_push_f32(const ds4hip_rows_push *p, uint8_t *codes, int8_t *sexp, uint16_t *tail,
                                          int head_dim, int n_rot, void *stream) {
    if (!p || !shape_ok(head_dim, n_rot) || p->f32_n < 0 || (p->f32_n && (!p->f32_src || !p->f32_dst ||
                                                                       !p->f32_dst_rows || p->f32_width <= 0 ||
                                                                       p->f32_width % 4)))
        return ds4hip_set_last_error(kEINVAL);
    RowsPushArgs A = {};
    A.p = *p;
    int blk = 0;
    for (int k = 0; k < 2; ++k) {
        if (p->fp8_n[k] < 0 ||
            (p->fp8_n[k] && (!p->fp8_src[k] || !p->fp8_dst[k] || !codes || !sexp || (n_rot > 0 && !tail))))
            return ds4hip_set_last_error(kEINVAL);
        blk += (p->fp8_n[k] + 3) / 4;
        A.blk[k] = blk;
    }
    blk += (p->f32_n + 3) / 4;
    A.blk[2] = blk;
    if (blk == 0) return 0;
    A.codes = codes;
    A.sexp = sexp;
    A.tail = tail;
    A.head_dim = head_dim;
    A.n_rot = n_rot;
    hipLaunchKernelGGL(rows_push_kernel, dim3(blk), dim3(256), 0, (hipStream_t)stream, A);
    return ds4hip_set_last_error(hip_status(hipGetLastError()));
}
