// C ABI entry points (declared in include/nvm_moe.h): argument validation,
// workspace layout and the launch sequence of the MoE block.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <mutex>
#include <string>

#include "internal.h"
#include "nvm_model.h"
#include "nvm_moe.h"

namespace {
thread_local std::string g_err;
}  // namespace

namespace nvm {
int set_error(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}
}  // namespace nvm

namespace {

int (*const fail)(int, const char *, ...) = nvm::set_error;

#define NVM_TRY_HIP(expr)                                                              \
  do {                                                                                 \
    const hipError_t e_ = (expr);                                                      \
    if (e_ != hipSuccess) return fail(NVM_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_)); \
  } while (0)

#define NVM_REQUIRE(cond, ...)                                  \
  do {                                                          \
    if (!(cond)) return fail(NVM_ERR_INVALID, __VA_ARGS__);     \
  } while (0)

#define NVM_SUPPORTED(cond, ...)                                \
  do {                                                          \
    if (!(cond)) return fail(NVM_ERR_UNSUPPORTED, __VA_ARGS__); \
  } while (0)

constexpr int64_t kMaxExperts = nvm::kMaxExperts;
constexpr int kMaxTopK = 64;
// reduction dimensions the product kernels are built and tested for
constexpr int64_t kMaxProductK = 8192;

// Largest buffer the kernels' 32-bit buffer descriptors and offsets address.
constexpr int64_t k2GiB = 0x7FFF0000ll;

// Bump allocator over the caller's workspace: slices at 256-byte aligned
// device addresses, whatever the alignment of the workspace itself.  Sizes
// (Carve over nullptr) include 256 bytes of slack for the first slice's
// alignment.
struct Carve {
  size_t off = 0;
  char *base;
  explicit Carve(void *b) : base((char *)b) {}
  template <class T>
  T *take(size_t count) {
    off = (size_t)((((uintptr_t)base + off + 255) & ~(uintptr_t)255) - (uintptr_t)base);
    T *p = base ? (T *)(base + off) : nullptr;
    off += count * sizeof(T);
    return p;
  }
  // bytes a workspace needs for the slices taken so far (base == nullptr)
  size_t bytes() const { return ((off + 255) & ~(size_t)255) + 256; }
};

int check_quant(int group_size, int bits, int dtype) {
  NVM_SUPPORTED(bits == 4, "bits must be 4 (got %d)", bits);
  NVM_SUPPORTED(group_size == 64 || group_size == 128, "group_size must be 64 or 128 (got %d)",
                group_size);
  NVM_REQUIRE(dtype == NVM_DTYPE_F16 || dtype == NVM_DTYPE_BF16, "dtype must be f16 or bf16");
  return NVM_OK;
}

// Decode GEMV or prefill GEMM for `pairs` routed rows over E experts with a
// reduction dimension of K.  Shapes the GEMV does not tile run on the GEMM.
bool use_decode(int regime, int64_t pairs, int64_t E, int64_t K) {
  if (!nvm::gemv_supports((int)K)) return false;
  if (regime == NVM_REGIME_DECODE) return true;
  if (regime == NVM_REGIME_PREFILL) return false;
  return pairs <= 8 * E;  // up to 8 routed rows per expert on average
}

// Shapes the expert products handle: K dims in whole 64-wide groups, output
// rows in whole 16-row MFMA tiles (both implied by multiples of 64).
int check_products(int64_t H, int64_t I, int64_t E, int top_k, int group_size, int bits,
                   int dtype, int regime) {
  if (int r = check_quant(group_size, bits, dtype)) return r;
  NVM_REQUIRE(H > 0 && I > 0 && E > 0, "moe: bad shape");
  NVM_REQUIRE(H % 64 == 0 && H % group_size == 0,
              "moe: hidden %lld must be a multiple of 64 and of group_size", (long long)H);
  NVM_REQUIRE(I % 64 == 0 && I % group_size == 0,
              "moe: intermediate %lld must be a multiple of 64 and of group_size", (long long)I);
  NVM_SUPPORTED(E <= kMaxExperts, "moe: at most %lld experts", (long long)kMaxExperts);
  NVM_REQUIRE(top_k >= 1 && top_k <= E, "moe: top_k=%d outside [1, E=%lld]", top_k,
              (long long)E);
  NVM_SUPPORTED(top_k <= kMaxTopK, "moe: top_k at most %d", kMaxTopK);
  NVM_REQUIRE(regime >= NVM_REGIME_AUTO && regime <= NVM_REGIME_PREFILL, "moe: bad regime %d",
              regime);
  NVM_SUPPORTED(H <= kMaxProductK && I <= kMaxProductK, "moe: H and I at most %lld",
                (long long)kMaxProductK);
  return NVM_OK;
}

// Workspace of the whole block; with base == nullptr only the size is computed.
struct MoeWs {
  double *partial;
  int32_t *ids;
  uint16_t *scores;
  int32_t *offsets, *sorted, *counts;
  unsigned *done;
  uint16_t *h, *down;
  uint8_t *xsh, *hsh;  // group shifts of the prefill GEMMs' fp16 copies of x and h
  // the float32 half sums of the down reduction [2][T*k][H] (decode batches
  // of at most 64 tokens), and whether the products left the down output
  // there (launch_gemv3_fused_down) instead of in `down`
  float *dpart;
  bool split;
  size_t bytes;
};

MoeWs carve_moe(void *base, int64_t T, int64_t H, int64_t I, int64_t E, int k) {
  Carve c(base);
  MoeWs w;
  const int64_t N = T * k;
  const int splits =
      std::max(nvm::route_workspace_splits(T, H, E), nvm::decode_route_splits(T, H, E));
  w.partial = c.take<double>((size_t)splits * T * E);
  w.ids = c.take<int32_t>(N);
  w.scores = c.take<uint16_t>(N);
  w.offsets = c.take<int32_t>(E + 1);
  w.sorted = c.take<int32_t>(N);
  w.counts = c.take<int32_t>((size_t)nvm::dispatch_workspace_bytes(N, E) / sizeof(int32_t));
  w.done = c.take<unsigned>(1);
  w.h = c.take<uint16_t>((size_t)N * I);
  w.down = c.take<uint16_t>((size_t)N * H);
  w.xsh = c.take<uint8_t>((size_t)T * (H / 64));
  w.hsh = c.take<uint8_t>((size_t)N * (I / 64));
  // (forward_fuses_products needs them; T <= 64)
  w.dpart = T <= 64 && nvm::fused_route_supports(T, E, k) ? c.take<float>((size_t)2 * N * H)
                                                          : nullptr;
  w.split = false;
  w.bytes = c.bytes();
  return w;
}

// Routing then dispatch: one single-block launch finalises and sorts decode
// batches; batches the int8 router takes are routed whole in one launch and
// sorted in another (without probabilities, E <= 128); other batches
// finalise per token and sort over blocks.  xh (bf16 x; may be NULL): where
// the whole-routing launch may also store the fp16 copy of x (with its group
// shifts in xsh) that launch_act_to_f16 makes; *xh_done says whether it did.
int run_route_dispatch(int dtype, const void *x, int64_t T, int64_t H, const uint32_t *wr,
                       const void *sr, const void *br, int64_t E, int gs, int k, int norm,
                       void *probs, int32_t *ids, void *scores, int32_t *offsets, int32_t *sorted,
                       double *partial, int32_t *counts, unsigned *done, hipStream_t st,
                       void *xh = nullptr, uint8_t *xsh = nullptr, bool *xh_done = nullptr) {
  if (xh_done) *xh_done = false;
  if (!probs && !nvm::route_fused_dispatch(T, k) && nvm::route_i8_fin_supports(T, H, E, gs, k)) {
    // the histograms [T/16][E] live in the partial-logit workspace, which
    // this path does not use (T * E doubles at least)
    int32_t *hist = (int32_t *)partial;
    void *xo = dtype == NVM_DTYPE_BF16 ? xh : nullptr;
    NVM_TRY_HIP(nvm::launch_route_i8_fin(dtype, x, T, H, wr, sr, br, E, gs, k, norm, ids, scores,
                                         hist, xo, xo ? xsh : nullptr, st));
    NVM_TRY_HIP(nvm::launch_dispatch_hist(ids, T * k, E, hist, (T + 15) / 16, 16 * k, offsets,
                                          sorted, st));
    if (xh_done) *xh_done = xo != nullptr;
    return NVM_OK;
  }
  const int splits = nvm::route_splits(T, H, E);
  const bool fused = nvm::route_fused_dispatch(T, k);
  NVM_TRY_HIP(nvm::launch_route_partial(dtype, x, T, H, wr, sr, br, E, gs, false, partial, nullptr,
                                        fused ? done : nullptr, st));
  if (fused) {
    NVM_TRY_HIP(nvm::launch_route_finalize_dispatch(dtype, partial, splits, T, E, k, norm, probs,
                                                    ids, scores, offsets, sorted, done, st));
  } else {
    NVM_TRY_HIP(nvm::launch_route_finalize(dtype, partial, splits, T, E, k, norm, probs, ids,
                                           scores, st));
    NVM_TRY_HIP(nvm::launch_dispatch(ids, T * k, E, offsets, sorted, counts, st));
  }
  return NVM_OK;
}

int check_route(const void *x, int64_t T, int64_t H, const uint32_t *wr, const void *sr,
                const void *br, int64_t E, int group_size, int bits, int top_k, int dtype,
                const int32_t *ids, const void *scores) {
  if (int r = check_quant(group_size, bits, dtype)) return r;
  NVM_REQUIRE(x && wr && sr && br && ids && scores, "route: null pointer");
  NVM_REQUIRE(T >= 0 && H > 0 && E > 0, "route: bad shape");
  NVM_REQUIRE(H % group_size == 0, "route: H=%lld not divisible by group_size %d",
              (long long)H, group_size);
  NVM_SUPPORTED(E <= kMaxExperts, "route: at most %lld experts", (long long)kMaxExperts);
  NVM_REQUIRE(top_k >= 1 && top_k <= E, "route: top_k=%d outside [1, E=%lld]", top_k,
              (long long)E);
  NVM_SUPPORTED(top_k <= kMaxTopK, "route: top_k at most %d", kMaxTopK);
  // the router kernels address x and the router weights through 32-bit
  // buffer offsets
  NVM_SUPPORTED(T * H * 2 <= k2GiB && E * (H / 2) <= k2GiB,
                "route: activations of %lld bytes or router weights of %lld bytes exceed 2 GiB; "
                "split the batch", (long long)(T * H * 2), (long long)(E * (H / 2)));
  return NVM_OK;
}

int run_products(int dtype, bool decode, bool dual, nvm::GroupedArgs &g, int64_t pairs,
                 hipStream_t st) {
  // the kernels address activations through 32-bit buffer offsets
  NVM_SUPPORTED(g.act_rows * g.act_ld * 2 <= k2GiB,
                "expert products: activation buffer of %lld bytes exceeds 2 GiB; split the batch",
                (long long)(g.act_rows * g.act_ld * 2));
  if (decode) {
    NVM_TRY_HIP(nvm::launch_gemv(dtype, dual, g, st));
  } else {
    const int64_t max_tiles = pairs / nvm::kGemmBM + g.E;
    NVM_TRY_HIP(nvm::launch_gemm(dtype, dual, g, max_tiles, st));
  }
  return NVM_OK;
}

// Arguments of the gate/up product: sorted slot n reads token row
// sorted[n] / top_k of x and writes row n of h [pairs, I].
nvm::GroupedArgs gateup_args(const void *x, int64_t T, int64_t H, int64_t I, int64_t E,
                             int top_k, int group_size, const uint32_t *wg, const void *sg,
                             const void *bg, const uint32_t *wu, const void *su, const void *bu,
                             const int32_t *offsets, const int32_t *sorted, void *h) {
  nvm::GroupedArgs g{};
  g.act = (const uint16_t *)x;
  g.act_ld = H;
  g.act_rows = T;
  g.a_map = sorted;
  g.a_div = top_k;
  g.offsets = offsets;
  g.w0 = wg;
  g.s0 = (const uint16_t *)sg;
  g.b0 = (const uint16_t *)bg;
  g.w1 = wu;
  g.s1 = (const uint16_t *)su;
  g.b1 = (const uint16_t *)bu;
  g.R = (int)I;
  g.K = (int)H;
  g.gs = group_size;
  g.E = (int)E;
  g.out = (uint16_t *)h;
  g.o_map = nullptr;
  g.out_ld = I;
  return g;
}

// Arguments of the down product: sorted slot n reads row n of h and writes
// row sorted[n] (the flat pair index) of down [pairs, H].
nvm::GroupedArgs down_args(const void *h, int64_t n_pairs, int64_t H, int64_t I, int64_t E,
                           int group_size, const uint32_t *wd, const void *sd, const void *bd,
                           const int32_t *offsets, const int32_t *sorted, void *down) {
  nvm::GroupedArgs d{};
  d.act = (const uint16_t *)h;
  d.act_ld = I;
  d.act_rows = n_pairs;
  d.a_map = nullptr;
  d.a_div = 1;
  d.offsets = offsets;
  d.w0 = wd;
  d.s0 = (const uint16_t *)sd;
  d.b0 = (const uint16_t *)bd;
  d.R = (int)H;
  d.K = (int)I;
  d.gs = group_size;
  d.E = (int)E;
  d.out = (uint16_t *)down;
  d.o_map = sorted;
  d.out_ld = H;
  return d;
}

// The forward's decode down product with the combine in its epilogue (one
// block per 16 columns of y over every pair), for batches of at most
// kDownCombinePairs pairs: y is bit-identical to the down product followed
// by the combine, so the choice by batch size keeps every token's output
// independent of its batch.  It saves the combine launch, but its 128 blocks
// (H 2048) each stream every touched expert's 16 rows with one unit of ring
// per wavefront: one token's layer took 28.6 against 30.5 us, eight tokens'
// 62.7 against 56.9 us.  NVM_DOWN_COMBINE=0/1 overrides the choice.
constexpr int64_t kDownCombinePairs = 16;
bool use_down_combine(int regime, int64_t T, int64_t H, int64_t I, int64_t E, int top_k,
                      int group_size) {
  const int64_t N = T * top_k;
  if (!use_decode(regime, N, E, I) ||
      !nvm::gemv3_down_combine_supports((int)I, (int)H, (int)E, group_size, N, top_k))
    return false;
  const char *v = getenv("NVM_DOWN_COMBINE");
  if (v && (v[0] == '0' || v[0] == '1')) return v[0] == '1';
  return N <= kDownCombinePairs;
}

int run_down_combine(int dtype, const MoeWs &ws, const uint16_t *scores, int64_t T, int64_t H,
                     int64_t I, int64_t E, int top_k, int group_size, const uint32_t *wd,
                     const void *sd, const void *bd, void *y, nvm_stream_t stream) {
  nvm::GroupedArgs d = down_args(ws.h, T * top_k, H, I, E, group_size, wd, sd, bd, ws.offsets,
                                 ws.sorted, nullptr);
  d.c_scores = scores;
  d.c_y = (uint16_t *)y;
  d.c_k = top_k;
  NVM_TRY_HIP(nvm::launch_gemv3_down_combine(dtype, d, (hipStream_t)stream));
  return NVM_OK;
}

// The decode gate/up and down products in one launch (expert-major blocks,
// two per expert, each over one half of the down reduction): taken from one
// routed row per expert on average at the shapes it supports (B = 16: 74.7
// against 76.0 us for the dealt products; B = 8 leaves too many blocks
// idle).  y is bit-identical either way, so the choice keeps every token's
// output independent of its batch.
// NVM_FUSED_DOWN=0/1 overrides the choice (within the shapes it supports);
// NVM_GEMV_STATIC=0 turns it off with the other expert-major products.
bool use_fused_down(int64_t T, int64_t H, int64_t I, int64_t E, int top_k, int group_size) {
  if (!nvm::gemv3_fused_down_supports((int)H, (int)I, (int)H, (int)E, group_size, T, top_k))
    return false;
  const char *v = getenv("NVM_FUSED_DOWN");
  if (v && (v[0] == '0' || v[0] == '1')) return v[0] == '1';
  const char *st = getenv("NVM_GEMV_STATIC");
  if (st && st[0] == '0') return false;
  return T * top_k >= E;
}

// nvm_moe_forward runs the decode products as one launch (the decode branch
// of moe_stages with the half sums carved in the workspace).
bool forward_fuses_products(int64_t T, int64_t H, int64_t I, int64_t E, int top_k,
                            int group_size, int regime) {
  return T > 0 && T <= 64 && nvm::fused_route_supports(T, E, top_k) &&
         use_decode(regime, T * top_k, E, H) &&
         use_fused_down(T, H, I, E, top_k, group_size);
}

// Routing, dispatch and both expert products of the block (everything but
// the combine), on the caller's workspace; `scores` is where the routing
// scores went; with ws.split the down output is left as the float32 half
// sums ws.dpart (launch_combine_split).
int moe_stages(const void *x, int64_t T, int64_t H, int64_t I, int64_t E, int top_k,
               int norm_topk_prob, int group_size, int bits, int dtype, const uint32_t *wr,
               const void *sr, const void *br, const uint32_t *wg, const void *sg,
               const void *bg, const uint32_t *wu, const void *su, const void *bu,
               const uint32_t *wd, const void *sd, const void *bd, int32_t *ids_out,
               void *scores_out, int regime, void *workspace, size_t workspace_bytes,
               nvm_stream_t stream, MoeWs &ws, uint16_t *&scores, int first = 0,
               int last = 2);

// Workspace of nvm_moe_forward_noalloc: a file-scope device array, one copy
// per GPU, held until the process ends.  Host code never uses the array's
// name as an address: each device's copy is located once with
// hipGetSymbolAddress and that pointer is what the kernels receive.
constexpr size_t kScratchBytes = size_t(32) << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// The current device's copy of `scratch`, located on first use.
int scratch_for_current_device(void **out) {
  int dev = -1;
  NVM_TRY_HIP(hipGetDevice(&dev));
  NVM_SUPPORTED(dev >= 0 && dev < kMaxDevices, "moe_noalloc: device %d beyond %d", dev,
                kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    NVM_TRY_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    NVM_REQUIRE(p != nullptr, "moe_noalloc: no device address for the scratch array");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return NVM_OK;
}

}  // namespace

extern "C" {

int nvm_abi_version(void) { return NVM_ABI_VERSION; }

const char *nvm_last_error(void) { return g_err.c_str(); }

// Router-sized products (at most 512 outputs over at most 64 rows) run on the
// float64 router kernel, which rounds the exact sum once.  The rest (dense
// projections, prefill batches) run on the expert products as one expert with
// no offsets, accumulating in fp32 like the reference's kernel: exact float64
// sums are bound by the f64 matrix cores (2048 -> 512 over 4096 rows: 171 us
// against 48 us).
constexpr int64_t kExactOutMax = 512;
constexpr int64_t kExactRowsMax = 64;

int nvm_quantized_matmul(const void *scales, const void *biases, int group_size, int bits,
                         const void *a, const uint32_t *b, int transpose_b, void *out, int64_t M,
                         int64_t N, int64_t K, int dtype, nvm_stream_t stream) {
  if (int r = check_quant(group_size, bits, dtype)) return r;
  NVM_SUPPORTED(transpose_b == 1, "quantized_matmul: b must be transposed");
  NVM_REQUIRE(scales && biases && a && b && out, "quantized_matmul: null pointer");
  NVM_REQUIRE(M >= 0 && N > 0 && K > 0, "quantized_matmul: bad shape M=%lld N=%lld K=%lld",
              (long long)M, (long long)N, (long long)K);
  NVM_REQUIRE(N % group_size == 0, "quantized_matmul: N=%lld not divisible by group_size %d",
              (long long)N, group_size);
  if (M == 0) return NVM_OK;
  // (the product kernels address weights and activations through 32-bit
  // buffer offsets)
  // (the float64 path below has the same 32-bit limits)
  NVM_SUPPORTED(K * (N / 2) <= k2GiB && M * N * 2 <= k2GiB,
                "quantized_matmul: operands of more than 2 GiB (a %lld bytes, b %lld bytes); "
                "split the product", (long long)(M * N * 2), (long long)(K * (N / 2)));
  if ((K > kExactOutMax || M > kExactRowsMax) && K % 16 == 0 && N % 64 == 0 && N <= kMaxProductK) {
    nvm::GroupedArgs g{};
    g.act = (const uint16_t *)a;
    g.act_ld = N;
    g.act_rows = M;
    g.a_map = nullptr;
    g.a_div = 1;
    g.offsets = nullptr;  // one expert over all M rows
    g.w0 = b;
    g.s0 = (const uint16_t *)scales;
    g.b0 = (const uint16_t *)biases;
    g.R = (int)K;
    g.K = (int)N;
    g.gs = group_size;
    g.E = 1;
    g.out = (uint16_t *)out;
    g.o_map = nullptr;
    g.out_ld = K;
    // The GEMV streams the weights once per 16-row chunk; the GEMM once, but
    // a block runs all N/64 k-steps in sequence, so a grid of fewer blocks
    // than CUs leaves the GEMM latency-bound.  GEMV up to two chunks, and up
    // to 32 chunks while the GEMM grid would not fill the chip.
    const int64_t gemm_blocks = (M + nvm::kGemmBM - 1) / nvm::kGemmBM * ((K + 255) / 256);
    const bool decode = nvm::gemv_supports((int)N) &&
                        (M <= 32 || (M <= 512 && gemm_blocks < nvm::cu_count()));
    return run_products(dtype, decode, false, g, M, (hipStream_t)stream);
  }
  NVM_TRY_HIP(nvm::launch_route_partial(dtype, a, M, N, b, scales, biases, K, group_size, true,
                                        nullptr, out, nullptr, (hipStream_t)stream));
  return NVM_OK;
}

int nvm_route_workspace_size(int64_t T, int64_t H, int64_t E, size_t *bytes) {
  NVM_REQUIRE(bytes, "route_workspace_size: null output");
  NVM_REQUIRE(T >= 0 && H > 0 && E > 0, "route_workspace_size: bad shape");
  *bytes = sizeof(double) * (size_t)nvm::route_workspace_splits(T, H, E) * (size_t)T * (size_t)E;
  return NVM_OK;
}

int nvm_moe_route(const void *x, int64_t T, int64_t H, const uint32_t *wr, const void *sr,
                  const void *br, int64_t E, int group_size, int bits, int top_k,
                  int norm_topk_prob, int dtype, void *probs, int32_t *ids, void *scores,
                  void *workspace, size_t workspace_bytes, nvm_stream_t stream) {
  if (int r = check_route(x, T, H, wr, sr, br, E, group_size, bits, top_k, dtype, ids, scores))
    return r;
  if (T == 0) return NVM_OK;
  size_t need = 0;
  nvm_route_workspace_size(T, H, E, &need);
  if (!workspace || workspace_bytes < need)
    return fail(NVM_ERR_WORKSPACE, "route: workspace of %zu bytes needed", need);
  const int splits = nvm::route_splits(T, H, E);
  hipStream_t st = (hipStream_t)stream;
  NVM_TRY_HIP(nvm::launch_route_partial(dtype, x, T, H, wr, sr, br, E, group_size, false,
                                        (double *)workspace, nullptr, nullptr, st));
  NVM_TRY_HIP(nvm::launch_route_finalize(dtype, (const double *)workspace, splits, T, E, top_k,
                                         norm_topk_prob, probs, ids, scores, st));
  return NVM_OK;
}

int nvm_dispatch_workspace_size(int64_t n, int64_t E, size_t *bytes) {
  NVM_REQUIRE(bytes, "dispatch_workspace_size: null output");
  NVM_REQUIRE(n >= 0 && E > 0, "dispatch_workspace_size: bad shape");
  *bytes = (size_t)nvm::dispatch_workspace_bytes(n, E);
  return NVM_OK;
}

int nvm_moe_dispatch(const int32_t *ids, int64_t n, int64_t E, int32_t *expert_offsets,
                     int32_t *sorted_pairs, void *workspace, size_t workspace_bytes,
                     nvm_stream_t stream) {
  NVM_REQUIRE(expert_offsets && (n == 0 || (ids && sorted_pairs)), "dispatch: null pointer");
  NVM_REQUIRE(n >= 0 && E > 0, "dispatch: bad shape");
  NVM_SUPPORTED(E <= kMaxExperts, "dispatch: at most %lld experts", (long long)kMaxExperts);
  NVM_SUPPORTED(n < (1ll << 31), "dispatch: too many pairs");
  const size_t need = (size_t)nvm::dispatch_workspace_bytes(n, E);
  if (need && (!workspace || workspace_bytes < need))
    return fail(NVM_ERR_WORKSPACE, "dispatch: workspace of %zu bytes needed", need);
  NVM_TRY_HIP(nvm::launch_dispatch(ids, n, E, expert_offsets, sorted_pairs, workspace,
                                   (hipStream_t)stream));
  return NVM_OK;
}

int nvm_route_dispatch_workspace_size(int64_t T, int64_t H, int64_t E, int top_k, size_t *bytes) {
  NVM_REQUIRE(bytes, "route_dispatch_workspace_size: null output");
  NVM_REQUIRE(T >= 0 && H > 0 && E > 0 && top_k > 0, "route_dispatch_workspace_size: bad shape");
  Carve c(nullptr);
  c.take<double>((size_t)nvm::route_workspace_splits(T, H, E) * T * E);
  c.take<int32_t>((size_t)nvm::dispatch_workspace_bytes(T * top_k, E) / sizeof(int32_t));
  c.take<unsigned>(1);
  *bytes = c.bytes();
  return NVM_OK;
}

int nvm_moe_route_dispatch(const void *x, int64_t T, int64_t H, const uint32_t *wr,
                           const void *sr, const void *br, int64_t E, int group_size, int bits,
                           int top_k, int norm_topk_prob, int dtype, void *probs, int32_t *ids,
                           void *scores, int32_t *expert_offsets, int32_t *sorted_pairs,
                           void *workspace, size_t workspace_bytes, nvm_stream_t stream) {
  if (int r = check_route(x, T, H, wr, sr, br, E, group_size, bits, top_k, dtype, ids, scores))
    return r;
  NVM_REQUIRE(expert_offsets && sorted_pairs, "route_dispatch: null pointer");
  if (T == 0) return NVM_OK;
  size_t need = 0;
  nvm_route_dispatch_workspace_size(T, H, E, top_k, &need);
  if (!workspace || workspace_bytes < need)
    return fail(NVM_ERR_WORKSPACE, "route_dispatch: workspace of %zu bytes needed", need);
  Carve c(workspace);
  double *partial = c.take<double>((size_t)nvm::route_workspace_splits(T, H, E) * T * E);
  int32_t *counts =
      c.take<int32_t>((size_t)nvm::dispatch_workspace_bytes(T * top_k, E) / sizeof(int32_t));
  unsigned *done = c.take<unsigned>(1);
  return run_route_dispatch(dtype, x, T, H, wr, sr, br, E, group_size, top_k, norm_topk_prob,
                            probs, ids, scores, expert_offsets, sorted_pairs, partial, counts, done,
                            (hipStream_t)stream);
}

int nvm_grouped_linear_workspace_size(int64_t n, int64_t D, int64_t O, int64_t E, size_t *bytes) {
  NVM_REQUIRE(bytes, "grouped_linear_workspace_size: null output");
  NVM_REQUIRE(n >= 0 && E > 0, "grouped_linear_workspace_size: bad shape");
  (void)D;
  (void)O;
  Carve c(nullptr);
  c.take<int32_t>(E + 1);
  c.take<int32_t>(n);
  c.take<int32_t>((size_t)nvm::dispatch_workspace_bytes(n, E) / sizeof(int32_t));
  *bytes = c.bytes();
  return NVM_OK;
}

int nvm_grouped_expert_linear(const void *x, int64_t n, int64_t D, const uint32_t *w,
                              const void *s, const void *b, int64_t E, int64_t O, int group_size,
                              int bits, const int32_t *ids, int dtype, void *out, int regime,
                              void *workspace, size_t workspace_bytes, nvm_stream_t stream) {
  if (int r = check_quant(group_size, bits, dtype)) return r;
  NVM_REQUIRE(n >= 0 && D > 0 && O > 0 && E > 0, "grouped_linear: bad shape");
  NVM_REQUIRE(n == 0 || (x && w && s && b && ids && out), "grouped_linear: null pointer");
  NVM_REQUIRE(D % 64 == 0 && D % group_size == 0,
              "grouped_linear: D=%lld must be a multiple of 64 and of group_size",
              (long long)D);
  NVM_REQUIRE(O % 16 == 0, "grouped_linear: output dim %lld must be a multiple of 16",
              (long long)O);
  NVM_SUPPORTED(D <= kMaxProductK, "grouped_linear: D at most %lld", (long long)kMaxProductK);
  NVM_SUPPORTED(E <= kMaxExperts, "grouped_linear: at most %lld experts", (long long)kMaxExperts);
  if (n == 0) return NVM_OK;
  size_t need = 0;
  nvm_grouped_linear_workspace_size(n, D, O, E, &need);
  if (!workspace || workspace_bytes < need)
    return fail(NVM_ERR_WORKSPACE, "grouped_linear: workspace of %zu bytes needed", need);
  Carve c(workspace);
  int32_t *offsets = c.take<int32_t>(E + 1);
  int32_t *sorted = c.take<int32_t>(n);
  int32_t *counts = c.take<int32_t>((size_t)nvm::dispatch_workspace_bytes(n, E) / sizeof(int32_t));
  hipStream_t st = (hipStream_t)stream;
  NVM_TRY_HIP(nvm::launch_dispatch(ids, n, E, offsets, sorted, counts, st));
  nvm::GroupedArgs g{};
  g.act = (const uint16_t *)x;
  g.act_ld = D;
  g.act_rows = n;
  g.a_map = sorted;
  g.a_div = 1;
  g.offsets = offsets;
  g.w0 = w;
  g.s0 = (const uint16_t *)s;
  g.b0 = (const uint16_t *)b;
  g.R = (int)O;
  g.K = (int)D;
  g.gs = group_size;
  g.E = (int)E;
  g.out = (uint16_t *)out;
  g.o_map = sorted;
  g.out_ld = O;
  return run_products(dtype, use_decode(regime, n, E, D), false, g, n, st);
}

int nvm_moe_workspace_size(int64_t T, int64_t H, int64_t I, int64_t E, int top_k, size_t *bytes) {
  NVM_REQUIRE(bytes, "moe_workspace_size: null output");
  NVM_REQUIRE(T >= 0 && H > 0 && I > 0 && E > 0 && top_k > 0, "moe_workspace_size: bad shape");
  *bytes = carve_moe(nullptr, T, H, I, E, top_k).bytes;
  return NVM_OK;
}

int nvm_moe_expert_gateup(const void *x, int64_t T, int64_t H, int64_t I, int64_t E, int top_k,
                          int group_size, int bits, int dtype, const uint32_t *wg,
                          const void *sg, const void *bg, const uint32_t *wu, const void *su,
                          const void *bu, const int32_t *expert_offsets,
                          const int32_t *sorted_pairs, void *h, int regime,
                          nvm_stream_t stream) {
  if (int r = check_products(H, I, E, top_k, group_size, bits, dtype, regime)) return r;
  NVM_REQUIRE(x && wg && sg && bg && wu && su && bu && expert_offsets && sorted_pairs && h,
              "expert_gateup: null pointer");
  if (T == 0) return NVM_OK;
  nvm::GroupedArgs g = gateup_args(x, T, H, I, E, top_k, group_size, wg, sg, bg, wu, su, bu,
                                   expert_offsets, sorted_pairs, h);
  const int64_t N = T * top_k;
  return run_products(dtype, use_decode(regime, N, E, H), true, g, N, (hipStream_t)stream);
}

int nvm_moe_expert_down(const void *h, int64_t n_pairs, int64_t H, int64_t I, int64_t E,
                        int group_size, int bits, int dtype, const uint32_t *wd, const void *sd,
                        const void *bd, const int32_t *expert_offsets,
                        const int32_t *sorted_pairs, void *down, int regime,
                        nvm_stream_t stream) {
  if (int r = check_products(H, I, E, 1, group_size, bits, dtype, regime)) return r;
  NVM_REQUIRE(n_pairs >= 0, "expert_down: bad shape");
  NVM_REQUIRE(h && wd && sd && bd && expert_offsets && sorted_pairs && down,
              "expert_down: null pointer");
  if (n_pairs == 0) return NVM_OK;
  nvm::GroupedArgs d = down_args(h, n_pairs, H, I, E, group_size, wd, sd, bd, expert_offsets,
                                 sorted_pairs, down);
  return run_products(dtype, use_decode(regime, n_pairs, E, I), false, d, n_pairs,
                      (hipStream_t)stream);
}

int nvm_moe_combine(const void *down, const void *scores, int64_t T, int top_k, int64_t H,
                    int dtype, void *y, nvm_stream_t stream) {
  NVM_REQUIRE(dtype == NVM_DTYPE_F16 || dtype == NVM_DTYPE_BF16, "dtype must be f16 or bf16");
  NVM_REQUIRE(T >= 0 && top_k >= 1 && H > 0 && H % 8 == 0,
              "combine: bad shape (H must be a multiple of 8)");
  NVM_REQUIRE(T == 0 || (down && scores && y), "combine: null pointer");
  if (T == 0) return NVM_OK;
  NVM_TRY_HIP(nvm::launch_combine(dtype, down, scores, T, top_k, H, y, (hipStream_t)stream));
  return NVM_OK;
}

int nvm_moe_forward(const void *x, int64_t T, int64_t H, int64_t I, int64_t E, int top_k,
                    int norm_topk_prob, int group_size, int bits, int dtype, const uint32_t *wr,
                    const void *sr, const void *br, const uint32_t *wg, const void *sg,
                    const void *bg, const uint32_t *wu, const void *su, const void *bu,
                    const uint32_t *wd, const void *sd, const void *bd, void *y, int32_t *ids_out,
                    void *scores_out, int regime, void *workspace, size_t workspace_bytes,
                    nvm_stream_t stream) {
  NVM_REQUIRE(y || T == 0, "moe: null pointer");
  MoeWs ws{};
  uint16_t *scores = nullptr;
  const bool fdc = T > 0 && use_down_combine(regime, T, H, I, E, top_k, group_size);
  if (int r = moe_stages(x, T, H, I, E, top_k, norm_topk_prob, group_size, bits, dtype, wr, sr,
                         br, wg, sg, bg, wu, su, bu, wd, sd, bd, ids_out, scores_out, regime,
                         workspace, workspace_bytes, stream, ws, scores, 0, fdc ? 1 : 2))
    return r;
  if (T == 0) return NVM_OK;
  if (fdc) return run_down_combine(dtype, ws, scores, T, H, I, E, top_k, group_size, wd, sd, bd, y,
                                   stream);
  if (ws.split) {
    NVM_TRY_HIP(nvm::launch_combine_split(dtype, ws.dpart, scores, T, top_k, H, y,
                                          (hipStream_t)stream));
    return NVM_OK;
  }
  return nvm_moe_combine(ws.down, scores, T, top_k, H, dtype, y, stream);
}

int nvm_moe_forward_stage(int stage, const void *x, int64_t T, int64_t H, int64_t I, int64_t E,
                          int top_k, int norm_topk_prob, int group_size, int bits, int dtype,
                          const uint32_t *wr, const void *sr, const void *br,
                          const uint32_t *wg, const void *sg, const void *bg,
                          const uint32_t *wu, const void *su, const void *bu,
                          const uint32_t *wd, const void *sd, const void *bd, void *y,
                          int32_t *ids_out, void *scores_out, int regime, void *workspace,
                          size_t workspace_bytes, nvm_stream_t stream) {
  NVM_REQUIRE(stage >= 0 && stage <= 5, "moe_stage: stage %d outside [0, 5]", stage);
  NVM_REQUIRE(y || T == 0 || (stage != 3 && stage != 5), "moe_stage: null pointer");
  MoeWs ws{};
  uint16_t *scores = nullptr;
  // stage 4: both products as the forward launches them; 5: its combine
  const int first = stage == 4 ? 1 : stage == 5 ? 3 : stage;
  const int last = stage == 4 ? 2 : stage == 5 ? 3 : stage;
  if (int r = moe_stages(x, T, H, I, E, top_k, norm_topk_prob, group_size, bits, dtype, wr, sr,
                         br, wg, sg, bg, wu, su, bu, wd, sd, bd, ids_out, scores_out, regime,
                         workspace, workspace_bytes, stream, ws, scores, first, last))
    return r;
  if (T == 0 || (stage != 3 && stage != 5)) return NVM_OK;
  if (stage == 5 && ws.dpart && forward_fuses_products(T, H, I, E, top_k, group_size, regime)) {
    NVM_TRY_HIP(nvm::launch_combine_split(dtype, ws.dpart, scores, T, top_k, H, y,
                                          (hipStream_t)stream));
    return NVM_OK;
  }
  return nvm_moe_combine(ws.down, scores, T, top_k, H, dtype, y, stream);
}

int nvm_moe_forward_plan(int64_t T, int64_t H, int64_t I, int64_t E, int top_k, int group_size,
                         int regime, int *fused_products) {
  NVM_REQUIRE(fused_products, "moe_forward_plan: null output");
  NVM_REQUIRE(T >= 0 && H > 0 && I > 0 && E > 0 && top_k > 0, "moe_forward_plan: bad shape");
  *fused_products = forward_fuses_products(T, H, I, E, top_k, group_size, regime) ? 1 : 0;
  return NVM_OK;
}

int nvm_moe_scratch_bytes(size_t *bytes) {
  NVM_REQUIRE(bytes, "moe_scratch_bytes: null output");
  *bytes = kScratchBytes;
  // Locate the current device's array now, outside any graph capture (the
  // lookup may load the code object).  Without a usable device this is a
  // size query only; the first noalloc call then locates it.
  int dev = -1;
  if (hipGetDevice(&dev) == hipSuccess) {
    void *p = nullptr;
    if (int r = scratch_for_current_device(&p)) return r;
  } else {
    (void)hipGetLastError();
  }
  return NVM_OK;
}

int nvm_moe_forward_noalloc(const void *x, int64_t T, int64_t H, int64_t I, int64_t E, int top_k,
                            int norm_topk_prob, int group_size, int bits, int dtype,
                            const uint32_t *wr, const void *sr, const void *br,
                            const uint32_t *wg, const void *sg, const void *bg,
                            const uint32_t *wu, const void *su, const void *bu,
                            const uint32_t *wd, const void *sd, const void *bd, void *y,
                            int32_t *ids_out, void *scores_out, int regime, nvm_stream_t stream) {
  NVM_REQUIRE(T >= 0 && H > 0 && I > 0 && E > 0 && top_k > 0, "moe_noalloc: bad shape");
  if (T == 0) return NVM_OK;
  const size_t need = carve_moe(nullptr, T, H, I, E, top_k).bytes;
  NVM_SUPPORTED(need <= kScratchBytes,
                "moe_noalloc: %lld tokens need %zu bytes of workspace, more than the %zu-byte "
                "static scratch; use nvm_moe_forward with a workspace",
                (long long)T, need, kScratchBytes);
  void *ws = nullptr;
  if (int r = scratch_for_current_device(&ws)) return r;
  return nvm_moe_forward(x, T, H, I, E, top_k, norm_topk_prob, group_size, bits, dtype, wr, sr,
                         br, wg, sg, bg, wu, su, bu, wd, sd, bd, y, ids_out, scores_out, regime,
                         ws, kScratchBytes, stream);
}

int nvm_moe_forward_residual_norm(const void *x, int64_t T, int64_t H, int64_t I, int64_t E,
                                  int top_k, int norm_topk_prob, int group_size, int bits,
                                  int dtype, const uint32_t *wr, const void *sr, const void *br,
                                  const uint32_t *wg, const void *sg, const void *bg,
                                  const uint32_t *wu, const void *su, const void *bu,
                                  const uint32_t *wd, const void *sd, const void *bd,
                                  const void *h, const void *norm_w, float eps, void *h_out,
                                  void *x_out, int regime, void *workspace,
                                  size_t workspace_bytes, nvm_stream_t stream) {
  NVM_SUPPORTED(nvm::combine_residual_norm_supports(H),
                "moe_residual_norm: hidden %lld must be a multiple of 8, at most 8192",
                (long long)H);
  NVM_REQUIRE(T == 0 || (h && norm_w && h_out && x_out), "moe_residual_norm: null pointer");
  // the fused kernel moves rows in 16-byte pieces
  NVM_REQUIRE(((uintptr_t)h | (uintptr_t)norm_w | (uintptr_t)h_out | (uintptr_t)x_out) % 16 == 0,
              "moe_residual_norm: h, norm_w, h_out and x_out must be 16-byte aligned");
  MoeWs ws{};
  uint16_t *scores = nullptr;
  if (int r = moe_stages(x, T, H, I, E, top_k, norm_topk_prob, group_size, bits, dtype, wr, sr,
                         br, wg, sg, bg, wu, su, bu, wd, sd, bd, nullptr, nullptr, regime,
                         workspace, workspace_bytes, stream, ws, scores))
    return r;
  if (T == 0) return NVM_OK;
  NVM_TRY_HIP(nvm::launch_combine_residual_norm(
      dtype, ws.split ? (const void *)ws.dpart : (const void *)ws.down, scores, T, top_k, H, h,
      norm_w, eps, h_out, x_out, (hipStream_t)stream, ws.split));
  return NVM_OK;
}

}  // extern "C"

namespace {

int moe_stages(const void *x, int64_t T, int64_t H, int64_t I, int64_t E, int top_k,
               int norm_topk_prob, int group_size, int bits, int dtype, const uint32_t *wr,
               const void *sr, const void *br, const uint32_t *wg, const void *sg,
               const void *bg, const uint32_t *wu, const void *su, const void *bu,
               const uint32_t *wd, const void *sd, const void *bd, int32_t *ids_out,
               void *scores_out, int regime, void *workspace, size_t workspace_bytes,
               nvm_stream_t stream, MoeWs &ws, uint16_t *&scores, int first, int last) {
  if (int r = check_products(H, I, E, top_k, group_size, bits, dtype, regime)) return r;
  NVM_REQUIRE(T >= 0, "moe: bad shape");
  NVM_REQUIRE(x && wr && sr && br && wg && sg && bg && wu && su && bu && wd && sd && bd,
              "moe: null pointer");
  if (T == 0) return NVM_OK;
  // Every kernel of the block addresses x, its fp16 copy, h and the router
  // weights through 32-bit buffer offsets: refuse larger operands here,
  // before the first launch, so that no stage runs on a batch a later stage
  // would refuse.
  NVM_SUPPORTED(T * H * 2 <= k2GiB && T * top_k * I * 2 <= k2GiB && E * (H / 2) <= k2GiB,
                "moe: activations of %lld bytes, h of %lld bytes or router weights of %lld "
                "bytes exceed 2 GiB; split the batch",
                (long long)(T * H * 2), (long long)(T * top_k * I * 2), (long long)(E * (H / 2)));
  const size_t need = carve_moe(nullptr, T, H, I, E, top_k).bytes;
  if (!workspace || workspace_bytes < need)
    return fail(NVM_ERR_WORKSPACE, "moe: workspace of %zu bytes needed", need);
  ws = carve_moe(workspace, T, H, I, E, top_k);
  int32_t *ids = ids_out ? ids_out : ws.ids;
  scores = scores_out ? (uint16_t *)scores_out : ws.scores;
  const int64_t N = T * top_k;
  hipStream_t st = (hipStream_t)stream;
  // stages: 0 routing (and dispatch), 1 gate/up + SwiGLU, 2 down; each reads
  // what the one before it left in the workspace
  auto runs = [&](int s) { return first <= s && s <= last; };
  if (nvm::fused_route_supports(T, E, top_k) && use_decode(regime, N, E, H)) {
    // Decode batches: one launch of float64 partial logits, then the gate/up
    // product finalises the routing and sorts the pairs in every block's
    // prologue (block 0 stores ids, scores, offsets and the sorted pairs).
    if (runs(0))
      NVM_TRY_HIP(nvm::launch_route_partial_decode(dtype, x, T, H, wr, sr, br, E, group_size,
                                                   ws.partial, st));
    if (runs(1)) {
      nvm::GroupedArgs g{};
      g.act = (const uint16_t *)x;
      g.act_ld = H;
      g.act_rows = T;
      g.a_div = top_k;
      g.offsets = ws.offsets;
      g.w0 = wg;
      g.s0 = (const uint16_t *)sg;
      g.b0 = (const uint16_t *)bg;
      g.w1 = wu;
      g.s1 = (const uint16_t *)su;
      g.b1 = (const uint16_t *)bu;
      g.R = (int)I;
      g.K = (int)H;
      g.gs = group_size;
      g.E = (int)E;
      g.out = ws.h;
      g.out_ld = I;
      g.route_part = ws.partial;
      g.route_splits = nvm::decode_route_splits(T, H, E);
      g.route_norm = norm_topk_prob;
      g.r_ids = ids;
      g.r_scores = scores;
      g.r_offsets = ws.offsets;
      g.r_sorted = ws.sorted;
      if (runs(2) && ws.dpart && forward_fuses_products(T, H, I, E, top_k, group_size, regime)) {
        // both products in one launch; the combine adds the down halves
        g.d_w = wd;
        g.d_s = (const uint16_t *)sd;
        g.d_b = (const uint16_t *)bd;
        g.d_part = ws.dpart;
        g.d_R = (int)H;
        NVM_TRY_HIP(nvm::launch_gemv3_fused_down(dtype, g, st));
        ws.split = true;
        return NVM_OK;
      }
      if (int r = run_products(dtype, true, true, g, N, st)) return r;
    }
  } else {
    // Both products on the prefill GEMM, which computes in fp16: x is
    // converted once (into the down buffer, which only the down product
    // writes, later; by the routing launch where it can) and the gate/up
    // epilogue stores h converted, instead of every tile of every block
    // converting its rows again.  The values are the ones the GEMMs' staging
    // would make.
    const bool gemm_both =
        dtype == NVM_DTYPE_BF16 && !use_decode(regime, N, E, H) && !use_decode(regime, N, E, I);
    if (runs(0)) {
      bool xh_done = false;
      if (int r = run_route_dispatch(dtype, x, T, H, wr, sr, br, E, group_size, top_k,
                                     norm_topk_prob, nullptr, ids, scores, ws.offsets, ws.sorted,
                                     ws.partial, ws.counts, ws.done, st,
                                     gemm_both ? ws.down : nullptr, ws.xsh, &xh_done))
        return r;
      if (gemm_both && !xh_done)
        NVM_TRY_HIP(nvm::launch_act_to_f16(x, T * H, ws.down, ws.xsh, st));
    }
    if (gemm_both) {
      if (runs(1)) {
        nvm::GroupedArgs g = gateup_args(ws.down, T, H, I, E, top_k, group_size, wg, sg, bg, wu,
                                         su, bu, ws.offsets, ws.sorted, ws.h);
        g.act_h = 1;
        g.out_h = 1;
        g.act_sh = ws.xsh;
        g.out_sh = ws.hsh;
        if (int r = run_products(dtype, false, true, g, N, st)) return r;
      }
      if (runs(2)) {
        nvm::GroupedArgs d = down_args(ws.h, N, H, I, E, group_size, wd, sd, bd, ws.offsets,
                                       ws.sorted, ws.down);
        d.act_h = 1;
        d.act_sh = ws.hsh;
        if (int r = run_products(dtype, false, false, d, N, st)) return r;
      }
      return NVM_OK;
    }
    if (runs(1))
      if (int r = nvm_moe_expert_gateup(x, T, H, I, E, top_k, group_size, bits, dtype, wg, sg, bg,
                                        wu, su, bu, ws.offsets, ws.sorted, ws.h, regime, stream))
        return r;
  }
  if (runs(2))
    return nvm_moe_expert_down(ws.h, N, H, I, E, group_size, bits, dtype, wd, sd, bd, ws.offsets,
                               ws.sorted, ws.down, regime, stream);
  return NVM_OK;
}

}  // namespace
