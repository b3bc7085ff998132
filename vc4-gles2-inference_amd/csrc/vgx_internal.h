// Internal definitions shared by the libvgx translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <mutex>
#include <string>
#include <vector>

#include "vgx.h"

// ---------------------------------------------------------------------------
// Error plumbing: every entry point returns a status and records a message on
// the calling thread.
int vgx_fail(int status, const std::string& msg);
int vgx_hip_fail(hipError_t e, const char* what);

#define VGX_HIP(call)                                                        \
    do {                                                                     \
        hipError_t e_ = (call);                                              \
        if (e_ != hipSuccess) return vgx_hip_fail(e_, #call);                \
    } while (0)

#define VGX_LAUNCH_CHECK(what)                                               \
    do {                                                                     \
        hipError_t e_ = hipGetLastError();                                   \
        if (e_ != hipSuccess) return vgx_hip_fail(e_, what);                 \
    } while (0)

// ---------------------------------------------------------------------------
// Device-side description of one uploaded matrix.  The layout in HBM:
//   Q8: body rows x cols bytes, q8u8 (level + 128), 256-byte aligned rows
//       start at r*cols; wsr: rows f32 per-row scales (the value the kernel
//       multiplies the exact integer dot product by).
//   Q4: body rows of cols/2 nibble bytes (the container's), back to back
//       (the GEMV walks odd rows' chunks in reverse so a cache line two rows
//       share is loaded by one instruction), sm: rows x groups
//       u32 = (u16)s16 | (u16)m16 << 16 (parts 1 and 2 interleaved so one
//       4-byte load carries a group's scale and minimum), ps scalar.
//   T3: body = the container's texel grid, ceil(rows/2) texel rows of cols/8
//       texels (4 bytes: 8 columns of a row pair), each row padded with zero
//       codes to t3_rstride(cols) bytes; wsr: rows f32.
struct MatDev {
    const uint8_t* body;
    const float* wsr;
    const uint32_t* sm;
    float ps;
    int kind;
    int rows, cols;
    int out_off;  // row offset of this matrix in a group's concatenated output
    int blk_off;  // first block of this matrix in a group launch
    int pad0, pad1;
};

// Bytes from one q4 nibble row to the next in HBM.
__host__ __device__ constexpr int q4_rstride(int cols) { return cols / 2; }

// t3: 32-column chunks a texel row holds, and the bytes from one texel row
// (row pair) to the next in HBM.  The container's rows hold cols/8 texels
// (cols a multiple of 8); upload pads each to whole 32-column chunks of zero
// codes, so every kernel reads whole 16-byte chunks inside the row.
__host__ __device__ constexpr int t3_chunks(int cols) { return (cols + 31) / 32; }
__host__ __device__ constexpr int t3_rstride(int cols) { return t3_chunks(cols) * 16; }

struct vgx_ctx {
    int device = 0;
    int num_cu = 256;
    hipStream_t own = nullptr;
    hipStream_t stream = nullptr;
    // this device's address of the library's static key-slot array (the
    // no-allocation argmax entry point), resolved once per device at create
    unsigned long long* scratch_keys = nullptr;
    // split-K GEMM partial sums: the bound of every split launch, allocated
    // once at the first launch that splits, never regrown (freed at destroy)
    void* ws = nullptr;
    size_t ws_bytes = 0;
    std::mutex ws_mu;
};

struct vgx_mat {
    vgx_ctx* ctx = nullptr;
    MatDev d{};
    MatDev* d_dev = nullptr;  // the descriptor in device memory (single launches)
    size_t body_bytes = 0, plane_bytes = 0;  // the weight bytes a GEMV reads
    size_t body_alloc_bytes = 0;             // the body's allocation (q4 rows padded)
    void* body_alloc = nullptr;
    void* plane_alloc = nullptr;
};

struct vgx_group {
    vgx_ctx* ctx = nullptr;
    int n = 0, kind = 0, cols = 0, rows = 0, blocks = 0;
    int bpm = 0;  // tiles per matrix when all matrices have the same rows, else 0
    int lpr = 64, ri = 1;
    MatDev* d_dev = nullptr;  // n descriptors with out_off / blk_off filled
    std::vector<MatDev> host;  // the same descriptors, host copy
    // fused argmax: one best-key slot (u64) per workgroup of a launch
    unsigned long long* keys = nullptr;
    int nkeys = 0;
};

// ---------------------------------------------------------------------------
// Launch helpers implemented in vgx_gemv.hip.
// EPI_STORE_ARGMAX: EPI_STORE, and each workgroup stores the best key of its
// rows in its slot; a one-workgroup launch then reduces the slots to the
// first-maximum argmax of the whole output.
enum GemvEpi { EPI_STORE = 0, EPI_STORE_F32 = 1, EPI_GATE = 2, EPI_SPLIT = 3, EPI_STORE_ARGMAX = 4 };
// How the activation row reaches the kernel: q16, f32 (host quantisation on
// the device), or q16 through RMSNorm (every workgroup recomputes the
// statistics of x and stages rmsnorm(x, rw, eps)).
enum GemvX { X_I16 = 0, X_F32 = 1, X_RMS = 2 };

// Launches over at most this many matrices carry their descriptors by value in
// the kernel arguments, so no workgroup waits on a descriptor load.
constexpr int kInlineMats = 8;

// The tail of a greedy decode step, run by the argmax reduction when pos is
// set: hist[*pos + 1] = the token, ++*pos, and the token's q8 embedding row
// into x (the next step's input).
struct StepTail {
    int* pos;
    int* hist;
    int hist_len;
    const int8_t* emb;
    const float* emb_scale;
    int vocab, dim;
    int16_t* x;
};

struct GemvLaunch {
    MatDev md[kInlineMats];  // descriptors by value (nmat <= kInlineMats)
    MatDev md3;           // W3 by value (EPI_GATE)
    const MatDev* mats;   // device descriptors (nmat > kInlineMats)
    int nmat;
    int blocks;           // row tiles (kWaves * 64/lpr * ri units each)
    int grid;             // workgroups; each takes tiles b, b + grid, ...
    int bpm;              // tiles per matrix when every matrix has the same rows, else 0
    const int16_t* x;     // q16 input (or nullptr)
    const float* xf;      // f32 input (EPI_STORE_F32)
    const int16_t* res;   // residual (EPI_STORE / EPI_SPLIT)
    void* y;              // int16 or f32 output
    int gate;             // EPI_GATE: the second matrix is md3
    int hs;               // hidden store exponent (EPI_GATE)
    int split_chunk;      // first chunk of the second column half (EPI_SPLIT)
    int kind, cols, lpr, ri;
    const int16_t* rw;    // RMSNorm weight, q16 (X_RMS)
    float eps;            // RMSNorm epsilon (X_RMS)
    int* argmax_out;      // EPI_STORE_ARGMAX: the index
    unsigned long long* argmax_key;  // EPI_STORE_ARGMAX: one key slot per workgroup (nkeys of them)
    int nkeys;
    int total_rows;       // EPI_STORE_ARGMAX: length of the output
    StepTail tail;        // EPI_STORE_ARGMAX: the decode step's tail (pos nullptr: none)
};

int vgx_gemv_plan(int kind, int rows, int cols, int num_cu, int* lpr, int* ri, int* rows_per_block);
int vgx_gemv_launch(const GemvLaunch& L, hipStream_t s);
int vgx_argmax_launch(const int16_t* v, int n, int rows, int* out, hipStream_t s);
int vgx_dequant_launch(const MatDev& d, float* out, hipStream_t s);
