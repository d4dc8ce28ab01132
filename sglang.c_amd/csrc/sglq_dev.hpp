// sglq_dev.hpp — device-side definitions shared by the HIP translation units: the resident
// weight layout, vector types and error plumbing.  gfx950 (CDNA4) only.
//
// Device layout of one quantized weight W [N, K] ("tile layout"):
//   * N is cut into tiles of 16 columns (t = n / 16); K is re-indexed through kmap into device
//     positions k' (act-order groups made contiguous, each group padded to a multiple of 32) and
//     cut into MFMA steps of 32 (s = k' / 32).
//   * codes: for every (tile t, chunk c) one 1 KiB block = 64 lanes x 16 B, tiles outermost,
//     chunks of one tile contiguous.  Lane l carries column n = 16t + (l & 15) and
//     k' = 32 s + 8 (l >> 4) + i, i.e. exactly the B operand of v_mfma_f32_16x16x32_f16 for that
//     step.  4-bit kinds: a chunk is 4 steps, word j of the lane is step 4c+j, nibble i holds
//     k-offset i.  8-bit kind: a chunk is 2 steps, words (2j, 2j+1) are step 2c+j, byte b of
//     the pair holds k-offset b.
//   * U4/U8 meta, one entry per (tile, column, unit); a unit is a group when every group is a
//     whole number of chunks (META_GROUP, cpg chunks per group), else a step (META_STEP).
//     Entry = f16 scale | f16 -(1024 + zero) << 16 when every scale is f16-exact (4 bytes),
//     else f32 scale | f16 -(1024 + zero) << 32 (8 bytes).  nmeta units per column, padded to
//     a multiple of 4 (padding entries are zero), stored in quads: the entries of units
//     4v .. 4v+3 of the tile's 16 columns are contiguous, [t][v][16][4], so one wave's
//     entries of four consecutive units are one contiguous run (sglq_mrow / sglq_mofs).
//   * E2M1 meta: the e8m0 byte of every (column, step), nmeta bytes per column (padded to a
//     multiple of 16), in the same quads of 4-byte words (one word = the four steps of a
//     chunk): [t][v][16][16 bytes]; plus the largest byte per column (colexp), the reference
//     exponent of the prefill GEMM.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sglq_shim.h"

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

enum { SGLQ_META_GROUP = 0, SGLQ_META_STEP = 1, SGLQ_META_E8M0 = 2 };

struct sglq_dev {
  int dev;
  int kind;       // SGLQ_KIND_*
  int scf16;      // U4/U8 meta entries hold f16 scales (4 B) rather than f32 (8 B)
  int prescale;   // f16 scales with |s| in [2^-14, 128]: (q - z) * s is a normal f16 number
  int src;        // SGLQ_SRC_* it was built from
  int meta_mode;  // SGLQ_META_*
  int kident;     // kmap is the identity on [0, K) (no act-order, no padding inside K)
  int64_t N, K;
  int64_t ntile;   // ceil(N / 16)
  int64_t nsteps;  // device K / 32
  int64_t spc;     // steps per chunk (4 for 4-bit kinds, 2 for 8-bit)
  int64_t nchunk;  // nsteps / spc
  int64_t spg;     // steps per group
  int64_t cpg;     // chunks per group (META_GROUP)
  int64_t ngroups; // real groups
  int64_t nmeta;   // meta entries per column
  u32x4_t *codes;
  void *meta;
  int32_t *kmap;  // [nsteps * 32]
  int32_t *kinv;  // [K]
  uint8_t *colexp;  // E2M1: largest e8m0 byte (255 excluded) of every column, [ntile * 16]
  // decode GEMV split-K state, sized at build: partial sums [gv_split][16][N] and one arrival
  // counter per tile (every counter is back at 0 when a launch ends)
  int gv_split;    // most K ranges a launch splits over
  float *gv_part;
  int *gv_cnt;
  // prefill GEMM / MoE workspace (grown on demand)
  void *ws;
  size_t ws_bytes;
  // buffers of an MoE shared-expert pass owned by its gate/up handle (grown on demand; apart
  // from ws, which the forwards inside that pass use)
  void *aux;
  size_t aux_bytes;
  // buffers outgrown by ws / aux, kept until the handle is freed (graphs captured earlier may
  // still reference them)
  void **retired;
  int nretired, cap_retired;
  // MoE: host copy of the expert pointer table last uploaded into ws (re-uploaded on change)
  void *moe_tbl;
  size_t moe_tbl_bytes;
  void *moe_tbl_ws;
};

#define SGLQ_HIP(expr)                                                                    \
  do {                                                                                    \
    hipError_t e_ = (expr);                                                               \
    if (e_ != hipSuccess) {                                                               \
      sglq_log_error("HIP error %s at %s:%d: %s", hipGetErrorName(e_), __FILE__, __LINE__, \
                     #expr);                                                              \
      goto fail;                                                                          \
    }                                                                                     \
  } while (0)

static inline unsigned sglq_blocks(int64_t n, int threads) {
  return (unsigned)((n + threads - 1) / threads);
}

// Dynamic LDS beyond 64 KiB is enabled per kernel and per device: raises kernel f's limit to
// `bytes` on the current device once (*done keeps one bit per device; devices past 63 are
// raised on every call).  Returns false when the runtime refuses.
inline bool sglq_raise_lds(const void *f, int bytes, unsigned long long *done) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  const unsigned long long bit = dev < 64 ? 1ull << dev : 0;
  if (bit && (__atomic_load_n(done, __ATOMIC_ACQUIRE) & bit)) return true;
  if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess)
    return false;
  if (bit) __atomic_fetch_or(done, bit, __ATOMIC_ACQ_REL);
  return true;
}

// Grow d->ws / d->aux to at least `bytes` (device memory; an outgrown buffer stays allocated
// until the handle is freed, since a graph captured earlier may hold its address).
int sglq_aux_reserve(sglq_dev *d, size_t bytes);
int sglq_ws_reserve(sglq_dev *d, size_t bytes);

// Decode-GEMV launch (gemv.hip): C rows [0, M) with M <= 16.
int sglq_gemv(sglq_dev *d, const void *A, int dt, int64_t lda, int64_t M, const float *bias,
              float *C, int64_t ldc, hipStream_t st);
// One-row decode GEMV (gemv_row.hip): 1 = launched, 0 = not applicable to this weight / row
// (the caller takes sglq_gemv), -1 = launch error.
int sglq_gemv_row(const sglq_dev *d, const void *A, int dt, const float *bias, float *C,
                  hipStream_t st);
// Grouped MoE decode GEMV on the one-row kernel (gemv_row.hip) for npairs = tokens x slots
// routing pairs read straight from the routing: pair j (expert ids[j], empty if outside
// [0, nexp)) writes C row j; grp 1 multiplies token row j / slots of A (lda), grp 2
// silu(A[j][:K]) * A[j][kcols:] (f32, lda) and also writes cout[t] (ldo) = the slot-order
// weighted sum (weights cw) of token t's rows; grp 3 (one token, at most 8 slots) writes only
// cout, combining the slots inside each tile's workgroup.  _ok: whether the weights and rows
// qualify.
// 1 = launched, 0 = not applicable, -1 = error.
int sglq_gemv_row_grouped_ok(const sglq_dev *d, int grp, const void *A, int dt, int64_t lda,
                             int kcols);
int sglq_gemv_row_grouped(const sglq_dev *d, const void *const *codes_e,
                          const void *const *meta_e, const int32_t *ids, int npairs, int slots,
                          int nexp, int grp, const void *A, int dt, int64_t lda, int kcols,
                          float *C, int64_t ldc, const float *cw, float *cout, int64_t ldo,
                          hipStream_t st);
// Kernels behind the host-buffer entry points (int8.hip), launched on st.
int sglq_launch_quant_rows_i8(const float *x, int8_t *q, float *scales, int64_t rows,
                              int64_t dim, hipStream_t st);
int sglq_launch_dequant_row_i8(const int8_t *q, float scale, float *o, int64_t n,
                               hipStream_t st);
int sglq_launch_matmul_nt(const float *A, const float *W, const float *bias, float *C,
                          int64_t M, int64_t N, int64_t K, hipStream_t st);
// Forward on an optional caller workspace for the prefill GEMM (gemv.hip; see there).
int sglq_forward_ws(sglq_dev *d, const void *A, int dt, int64_t M, const float *bias, float *C,
                    void *stream, void *ws, size_t ws_bytes);
// Prefill GEMM launch (gemm.hip): any M; grows the handle's workspace on first use at a size.
int sglq_gemm(sglq_dev *d, const void *A, int dt, int64_t lda, int64_t M, const float *bias,
              float *C, int64_t ldc, hipStream_t st);
// The same GEMM on a caller-provided workspace of at least sglq_gemm_ws_bytes bytes
// (256-byte aligned); allocates nothing.
size_t sglq_gemm_ws_bytes(const sglq_dev *d, int dt, int64_t M);
int sglq_gemm_ws(const sglq_dev *d, const void *A, int dt, int64_t lda, int64_t M,
                 const float *bias, float *C, int64_t ldc, void *ws, hipStream_t st);

// Grouped-GEMM building blocks (gemm.hip), used by the MoE path.
constexpr int SGLQ_GEMM_BM = 128;  // rows per GEMM row block
constexpr int SGLQ_MOE_BM = 64;    // rows per MoE row block (all of one expert)
struct sglq_group {               // per-expert weights (device arrays) + device row-block table
  const void *const *codes;       // [n_exp] u32x4_t*
  const void *const *meta;        // [n_exp]
  const uint8_t *const *colexp;   // [n_exp] (MXFP4)
  const int *segs;                // [max blocks][4] {expert, first row, rows, 0}
  const int *nseg;                // blocks in use (device scalar)
  int swiglu;                     // gate/up weights [2 mi, K]: mi > 0 = C gets silu(g) * u
  int *rowmax;                    // with swiglu: per-row max |C| bits (atomic max, preset 0)
  // one token (decode GEMVs only): segments straight from its routing, slot j = segment
  // {ids[j], row j, 1 row} when 0 <= ids[j] < nexp (segs, nseg and the row map are not used)
  const int32_t *ids;
  int nid, nexp;
};
// A operands of Mpad rows into aop (sglq_aop_bytes) + row exponents; mode 0 dense rows,
// 1 rows gathered through rowmap (-1 = zero row), 2 silu(A[m][k]) * A[m][kcols + k] (f32 A).
// rowmax (optional): per-row max |a| bits already known (the row exponents are derived from
// them and written to rowexp instead of a pass over the rows).
int sglq_prep_a(const sglq_dev *d, int mode, const void *A, int dt, int64_t lda, int64_t M,
                int64_t Mpad, const int32_t *rowmap, int kcols, int split, void *aop,
                int *rowexp, hipStream_t st, const int *rowmax = nullptr);
// the prefill GEMM of this weight runs the LDS-dequant kernel (needed for a fused SwiGLU)
bool sglq_gemm_lds_direct(const sglq_dev *d);
size_t sglq_aop_bytes(const sglq_dev *d, int64_t Mpad, int split);
// nblk row blocks (dense: block b = rows [128b, 128b+128); grouped: from grp->segs).
int sglq_gemm_run(const sglq_dev *d, const sglq_group *grp, const void *aop, const int *rowexp,
                  int64_t M, int64_t Mpad, int64_t nblk, int split, const float *bias, float *C,
                  int64_t ldc, float *part, hipStream_t st);
// Grouped decode GEMV (MoE): one launch over the row segments of grp (each <= max_rows rows of
// one expert, at most max_segs of them), activation rows per amode (0 A row r, 1 A row
// rowmap[r], 2 silu(A[r][k]) * A[r][kcols + k] with f32 A; A has a_rows rows).  Only when every workgroup can take
// all of K (sglq_gemv_grouped_fits).
int sglq_gemv_grouped_fits(const sglq_dev *d, int64_t max_rows, int split);
// The one-token MoE decode can take its segments straight from the routing (no routing
// kernel): both grouped launches take the wave-staged kernel and the down launch fuses the
// combine.  h: token row (h_dtype, E elements); gu: the gate/up output [k][2 mi] (f32).
int sglq_moe_direct_ok(const sglq_dev *gate_up, const sglq_dev *down, const void *h,
                       int h_dtype, int64_t E, const void *gu, int64_t k, int64_t mi);
// cmb (optional, one token): the down launch also forms out[n] = sum_j wts[j] * C[pos[j]][n]
// in slot order when its kernel can (then *cmb->done is set to 1, else left alone).
struct sglq_combine {
  const int32_t *pos;
  const float *wts;
  int k;
  float *out;
  int *done;
};
int sglq_gemv_grouped(const sglq_dev *d, const struct sglq_group *grp, int64_t max_rows,
                      int64_t max_segs, const void *A, int dt, int64_t a_rows, int64_t lda,
                      int amode, const int32_t *rowmap, int kcols, float *C, int64_t ldc,
                      hipStream_t st, const sglq_combine *cmb = nullptr);
// Picks the decode GEMV split for a freshly built weight and allocates its state.
int sglq_gemv_setup(sglq_dev *d);

// Meta entry (tile t, column n16 of the tile, unit u) = row base + offset, in entries (4 or 8
// bytes; for E2M1 4-byte words, u = chunk, nm = nmeta / 4); nm = entries per column.
__host__ __device__ __forceinline__ int64_t sglq_mrow(int64_t t, int n16, int64_t nm) {
  return t * nm * 16 + n16 * 4;
}
__host__ __device__ __forceinline__ int64_t sglq_mofs(int64_t u) { return (u >> 2) * 64 + (u & 3); }
// e8m0 byte of (tile t, column n16, step s), nmeta bytes per column
__host__ __device__ __forceinline__ int64_t sglq_ebyte(int64_t t, int n16, int64_t s,
                                                      int64_t nmeta) {
  return t * nmeta * 16 + (s >> 4) * 256 + n16 * 16 + (s & 15);
}

// silu(g) = g / (1 + e^-g) (reference src/deepseek.c:662-663) with the hardware exponential
// and reciprocal (v_exp_f32 on -g log2(e), v_rcp_f32): about 1e-6 relative error against
// the libm form, which costs ~20 VALU per element (exp range reduction and an IEEE divide).
// The MoE blocks are compared with the reference within 1e-3; routing scores keep libm expf.
__device__ __forceinline__ float sglq_silu(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * 1.44269504088896341f));
}

__device__ __forceinline__ float sglq_e2m1_value(uint32_t c) {
  // reference src/qweight.c:325-329
  const float mag[8] = {0.f, 0.5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f};
  const float v = mag[c & 7];
  return (c & 8) ? -v : v;
}
