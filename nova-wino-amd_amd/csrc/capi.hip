// C-ABI of libnova_winograd.so and the per-handle host runtime.
//
// The handle replaces the reference's NovaWinogradF63 / NovaWinogradFused
// host classes (/root/reference/csrc/nova_winograd.hip:456-611,
// /root/reference/csrc/nova_winograd_fused.hip:446-607): it owns the
// Winograd-domain filter U (product layout [64][K][Cp], plus its MFMA
// fragment-ordered copy for the fused kernels) and a grow-only workspace,
// launches on a caller-selected stream in the caller-selected activation
// layout, and picks the fused or the 3-pass pipeline per call. Errors are
// recorded per thread instead of exiting the process.
#include <cstdarg>
#include <cstdio>
#include <algorithm>
#include <cstring>
#include <functional>
#include <mutex>
#include <vector>

#include "../../include/nova_winograd.h"
#include "nova_internal.h"

namespace nova {

KernelEvents& kernel_events() {
    static thread_local KernelEvents ev;
    return ev;
}

static thread_local int g_err = 0;
static thread_local char g_msg[512] = "";

void set_error(int code, const char* fmt, ...) {
    g_err = code;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
    va_end(ap);
}

namespace {

constexpr uint32_t kMagic = 0x4e4f5641u;  // "NOVA"
// V + M bytes per window of the windowed three-pass path: the reference's
// 4 MiB L2 budget (/root/reference/tests/test_bp_tiled.hip:613-614).
constexpr int64_t kDefaultWindowBytes = (int64_t)4 << 20;

// Kernel kinds for per-kernel timing.
enum Kind { kKindInput = 0, kKindGemm = 1, kKindOutput = 2, kKindFused = 3, kNumKinds = 4 };

// Optional per-kernel timing: every kernel a forward launches records its own
// start and end into a pair of hipEvents (its dispatch packet's timestamps,
// see KernelEvents), so a pair times the kernel alone. Off by default (zero
// overhead); the event pool grows on demand up to kMaxEvents.
struct Profiler {
    static constexpr size_t kMaxEvents = 2 * 3 * 4096;  // 4096 three-kernel forwards
    bool on = false;
    std::vector<hipEvent_t> pool;
    size_t next = 0;
    struct Span {
        int kind;
        size_t e0, e1;
    };
    std::vector<Span> spans;
    const char* names[kNumKinds] = {"", "", "", ""};
    // last launch of each kind (first sub-batch), re-issued by replay()
    std::function<hipError_t()> last[kNumKinds];

    bool grow() {
        const size_t want = std::min(kMaxEvents, std::max<size_t>(64, 2 * pool.size()));
        while (pool.size() < want) {
            hipEvent_t e;
            if (hipEventCreate(&e) != hipSuccess) return false;
            pool.push_back(e);
        }
        return true;
    }
    // Arms the calling thread's kernel events for the next launch; returns the
    // index of the start event, or SIZE_MAX when disabled or exhausted.
    size_t arm() {
        if (!on) return SIZE_MAX;
        if (next + 2 > pool.size() && (pool.size() >= kMaxEvents || !grow())) return SIZE_MAX;
        if (next + 2 > pool.size()) return SIZE_MAX;
        kernel_events() = KernelEvents{pool[next], pool[next + 1]};
        next += 2;
        return next - 2;
    }
    // After the launch: records the kernel's name for its kind and keeps the
    // span if the kernel took the events.
    void done(int kind, size_t e0, const char* name) {
        names[kind] = name;
        if (e0 == SIZE_MAX) return;
        if (kernel_events().start != nullptr || kernel_events().stop != nullptr) {
            // a launch did not take its events: no span
            kernel_events() = KernelEvents{};
            return;
        }
        spans.push_back({kind, e0, e0 + 1});
    }
};

struct Handle {
    uint32_t magic = kMagic;
    int K = 0, C = 0, Cp = 0;
    uint16_t* U = nullptr;
    size_t U_cap = 0;  // bytes
    uint16_t* Uf = nullptr;  // U in MFMA fragment order (fused kernels)
    size_t Uf_cap = 0;       // bytes
    bool uf_ready = false;   // Uf holds the current weights' fragments
    uint16_t* Uw = nullptr;  // U in 1 KB operand blocks (two-pass kernel, GEMV-like GEMMs)
    size_t Uw_cap = 0;       // bytes
    bool uw_ready = false;   // Uw holds the current weights' blocks
    void* ws = nullptr;
    size_t ws_cap = 0;  // bytes
    unsigned* cnt = nullptr;  // fused-kernel arrival counters, zero between launches
    size_t cnt_cap = 0;       // counters
    hipStream_t stream = nullptr;
    int path_pref = 0;  // 0 auto, 1 three-pass, 2 fused rows, 3 fused block, 4 windowed,
                        // 5 small fused, 6 two-pass, 7 input transform in the products
    int64_t window_bytes = kDefaultWindowBytes;  // V + M per window of the windowed path
    Epilogue ep;        // bias / residual / ReLU applied by every forward
    int nhwc = 0;       // 1: x and y are NHWC (channels last)
    int last_path = 0;
    int cus = 256;  // compute units of the device the weights were set on
    int device = 0;  // that device
    bool ready = false;
    Profiler prof;
    hipEvent_t order_ev = nullptr;  // orders a new stream after the previous one
};

// True when s is being captured into a graph (or its state cannot be read).
bool is_capturing(hipStream_t s) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &st) != hipSuccess) {
        (void)hipGetLastError();
        return true;
    }
    return st != hipStreamCaptureStatusNone;
}

Handle* as_handle(nova_handle_t h, const char* fn) {
    Handle* H = static_cast<Handle*>(h);
    if (H == nullptr || H->magic != kMagic) {
        set_error(kErrInvalidArgument, "%s: invalid handle", fn);
        return nullptr;
    }
    return H;
}

bool hip_ok(hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    set_error(e == hipErrorOutOfMemory ? kErrOutOfMemory : kErrHip, "%s: %s", what,
              hipGetErrorString(e));
    return false;
}

void reference_tiling(int H, int W, int pad, int* nh, int* nw, int* Ho, int* Wo) {
    // /root/reference/csrc/nova_winograd.hip:617-631: pad the output extent
    // by n-1 = 7 and round (extent - 8) up to a multiple of 6.
    const int m = 6, n = 8;
    *Ho = H + 2 * pad - 2;
    *Wo = W + 2 * pad - 2;
    int hp = *Ho + n - 1, wp = *Wo + n - 1;
    hp += (m - (hp - n) % m) % m;
    wp += (m - (wp - n) % m) % m;
    *nh = (hp - n) / m + 1;
    *nw = (wp - n) / m + 1;
}

bool ensure_ws(Handle* H, size_t bytes) {
    if (bytes <= H->ws_cap) return true;
    if (H->ws) {
        if (!hip_ok(hipFree(H->ws), "hipFree(workspace)")) return false;
        H->ws = nullptr;
        H->ws_cap = 0;
    }
    // 25% headroom so that slowly growing batches do not reallocate each call
    const size_t want = bytes + bytes / 4;
    if (!hip_ok(hipMalloc(&H->ws, want), "hipMalloc(workspace)")) return false;
    H->ws_cap = want;
    return true;
}

// The fragment-ordered copy of U that the fused kernels read, built from U
// on the handle's stream the first time a fused path needs it for the
// current weights (set_weights builds it at once when the automatic choice
// can pick a fused kernel or one is forced, so a forward -- or a captured
// graph -- normally finds it ready). Layers that always run three-pass never
// hold it: for 1280 x 1280 channels that saves 210 MB per handle.
bool ensure_uf(Handle* H) {
    if (H->uf_ready) return true;
    const size_t need = (size_t)u_frag_elems(H->K, H->Cp) * sizeof(uint16_t);
    if ((int64_t)need >= ((int64_t)1 << 31)) {  // 32-bit offsets in the fused kernels
        set_error(kErrInvalidArgument, "fused filter copy of %lld bytes exceeds 2^31 - 1",
                  (long long)need);
        return false;
    }
    if (need > H->Uf_cap) {
        if (H->Uf) {
            if (!hip_ok(hipFree(H->Uf), "hipFree(Uf)")) return false;
            H->Uf = nullptr;
            H->Uf_cap = 0;
        }
        if (!hip_ok(hipMalloc(&H->Uf, need), "hipMalloc(Uf)")) return false;
        H->Uf_cap = need;
    }
    H->uf_ready = hip_ok(launch_u_frag(H->U, H->Uf, H->K, H->Cp, H->stream),
                         "filter fragment order");
    return H->uf_ready;
}

// U in 1 KB operand blocks (launch_u_wfrag), read by the two-pass kernel and
// by the three-pass GEMM at GEMV-like shapes (at most 32 tiles). Built like
// Uf: at set_weights when the automatic choice can pick path 6 or it is
// forced, else on the first forward that needs it.
bool ensure_uw(Handle* H) {
    if (H->uw_ready) return true;
    const size_t need = (size_t)u_frag_elems(H->K, H->Cp) * sizeof(uint16_t);
    if ((int64_t)need >= ((int64_t)1 << 31)) {  // 32-bit offsets in the two-pass kernel
        set_error(kErrInvalidArgument, "filter block copy of %lld bytes exceeds 2^31 - 1",
                  (long long)need);
        return false;
    }
    if (need > H->Uw_cap) {
        if (H->Uw) {
            if (!hip_ok(hipFree(H->Uw), "hipFree(Uw)")) return false;
            H->Uw = nullptr;
            H->Uw_cap = 0;
        }
        if (!hip_ok(hipMalloc(&H->Uw, need), "hipMalloc(Uw)")) return false;
        H->Uw_cap = need;
    }
    H->uw_ready = hip_ok(launch_u_wfrag(H->U, H->Uw, H->K, H->Cp, H->stream),
                         "filter two-pass order");
    return H->uw_ready;
}

// Counters of the fused kernel: zeroed once when (re)allocated; each launch
// returns every counter it uses to zero.
bool ensure_cnt(Handle* H, size_t count) {
    if (count <= H->cnt_cap) return true;
    if (H->cnt) {
        if (!hip_ok(hipFree(H->cnt), "hipFree(counters)")) return false;
        H->cnt = nullptr;
        H->cnt_cap = 0;
    }
    const size_t want = count + count / 4 + 64;
    if (!hip_ok(hipMalloc(&H->cnt, want * sizeof(unsigned)), "hipMalloc(counters)")) return false;
    if (!hip_ok(hipMemsetAsync(H->cnt, 0, want * sizeof(unsigned), H->stream),
                "hipMemsetAsync(counters)"))
        return false;
    H->cnt_cap = want;
    return true;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

struct Shape {
    int B, H, W, pad, Ho, Wo, nh, nw;
    int64_t BP;
};

bool make_shape(const Handle* Hd, int B, int H, int W, int pad, Shape* s, const char* fn) {
    if (B < 0 || H < 1 || W < 1 || pad < 0) {
        set_error(kErrInvalidArgument, "%s: bad shape B=%d H=%d W=%d pad=%d", fn, B, H, W, pad);
        return false;
    }
    s->B = B;
    s->H = H;
    s->W = W;
    s->pad = pad;
    s->Ho = H + 2 * pad - 2;
    s->Wo = W + 2 * pad - 2;
    if (s->Ho < 1 || s->Wo < 1) {
        set_error(kErrInvalidArgument, "%s: empty output for H=%d W=%d pad=%d", fn, H, W, pad);
        return false;
    }
    s->nh = tiles_min(s->Ho);
    s->nw = tiles_min(s->Wo);
    s->BP = (int64_t)B * s->nh * s->nw;
    const int cblocks = (Hd->Cp + 63) / 64, kblocks = (Hd->K + 63) / 64;
    if (s->nh > 65535 || (int64_t)B * cblocks > 65535 || (int64_t)B * kblocks > 65535) {
        set_error(kErrInvalidArgument, "%s: shape exceeds launch limits", fn);
        return false;
    }
    return true;
}

// Largest number of images per launch such that every buffer a kernel
// addresses (x, y, V, M) stays below 2 GB: the kernels use 32-bit byte
// offsets through buffer resources.
int64_t batch_chunk(const Handle* Hd, const Shape& s) {
    const int64_t P = (int64_t)s.nh * s.nw;
    const int64_t per_img = std::max(
        std::max(2 * (int64_t)Hd->C * s.H * s.W, 2 * (int64_t)Hd->K * s.Ho * s.Wo),
        2 * 64 * (int64_t)std::max(Hd->Cp, Hd->K) * P);
    return ((int64_t)1 << 31) / 2 / per_img;  // keep a 2x margin under INT_MAX
}

// Sub-batch size of a forward (every buffer a kernel addresses < 1 GB).
int64_t sub_batch(const Handle* Hd, const Shape& s) {
    return std::min<int64_t>(s.B, std::max<int64_t>(1, batch_chunk(Hd, s)));
}

bool fused_plan_for(const Handle* Hd, const Shape& s, FusedPlan* p) {
    const int64_t Bc = sub_batch(Hd, s);
    if (!fused_fits(Bc * Hd->C * s.H * s.W, u_frag_elems(Hd->K, Hd->Cp),
                    Bc * Hd->K * s.Ho * s.Wo))
        return false;
    return fused_plan((int)Bc, Hd->C, Hd->K, Hd->Cp, s.H, s.W, s.nh, s.nw, p);
}

bool fused_block_plan_for(const Handle* Hd, const Shape& s, FusedBlockPlan* p) {
    const int64_t Bc = sub_batch(Hd, s);
    if (!fused_fits(Bc * Hd->C * s.H * s.W, u_frag_elems(Hd->K, Hd->Cp),
                    Bc * Hd->K * s.Ho * s.Wo))
        return false;
    return fused_block_plan((int)Bc, Hd->C, Hd->K, Hd->Cp, s.H, s.W, s.nh, s.nw, p,
                            Hd->nhwc != 0);
}

// Pipeline for a forward: 1 three-pass, 2 fused (position-row split), 3 fused
// (tile block). A requested fused variant outside its envelope falls back to
// the three-pass pipeline.
// Images per launch of the windowed three-pass path: as many as keep V + M
// of the window within the handle's budget (at least one image; the
// reference windows tile ranges, this path whole images).
int64_t window_images(const Handle* Hd, const Shape& s) {
    const int64_t per_img = 2 * (int64_t)64 * (Hd->Cp + Hd->K) * s.nh * s.nw;
    return std::max<int64_t>(1, Hd->window_bytes / per_img);
}

bool fused_small_plan_for(const Handle* Hd, const Shape& s, FusedSmallPlan* p) {
    const int64_t Bc = sub_batch(Hd, s);
    if (!fused_fits(Bc * Hd->C * s.H * s.W, u_frag_elems(Hd->K, Hd->Cp),
                    Bc * Hd->K * s.Ho * s.Wo))
        return false;
    return fused_small_plan((int)Bc, Hd->C, Hd->K, Hd->Cp, s.nh, s.nw, Hd->cus, p);
}

// First tile of the short last 16-tile run of every image when the tile-block
// kernel should leave those tiles to the small-problem kernel (0: it takes
// every tile). A short run costs a workgroup as much as a full one; where
// the full runs alone need one round of workgroups less (one workgroup per
// CU), the short runs' tiles go to a second launch of the small-problem
// kernel (2 tiles x 16 output channels per workgroup, else 4 tiles, spread
// over every CU), while that launch has at most 2 workgroups per CU (1 at
// one 32-channel chunk): a round of the tile-block kernel costs ~19 us at
// two chunks, the small-problem launch of 2-tile workgroups ~11 us at 1.25
// per CU, ~17 at 2.5 and ~21 at 4, of 4-tile ones ~18 at 2. Whole forwards,
// graph of ten, us, one launch vs split: 64@56^2 batch 37 36.9 vs 31.3, 40
// 36.9 vs 32.2, 42 39.8 vs 32.5 (2 tiles); 74 55.8 vs 54.0, 80 56.1 vs 55.4
// (55.6 with 2 tiles), 85 59.4 vs 56.5, 112 74.6 vs 74.1, 128 78.4 vs 76.9
// (79.5 with 2 tiles), channels-last 78.3 vs 76.5 (4 tiles); 64@54^2 pad 2
// batch 43 (81 tiles) 39.6 vs 29.6; 32@56^2 batch 40 21.4 vs 18.9. Both
// kernels give the same bits for a tile.
int fused_tail_first(const Handle* Hd, const Shape& s, const FusedBlockPlan& bp,
                     FusedSmallPlan* tp) {
    const int P = s.nh * s.nw, full = P / 16;
    if (full == 0 || P % 16 == 0 || Hd->C > 64 || Hd->K > 64 || Hd->Cp > 64) return 0;
    const int64_t cus = Hd->cus;
    const int64_t g_full = (int64_t)s.B * full * bp.n_kblk;
    if ((g_full + cus - 1) / cus >= (bp.grid + cus - 1) / cus) return 0;
    const int64_t limit = (Hd->Cp > 32 ? 2 : 1) * cus;
    // 2 tiles per small-problem workgroup, else 4 (half the workgroups)
    for (int tiles : {2, 4})
        if (fused_small_plan(s.B, Hd->C, Hd->K, Hd->Cp, s.nh, s.nw, Hd->cus, tp, 16 * full,
                             tiles) &&
            tp->grid <= limit)
            return 16 * full;
    return 0;
}

// Layers the automatic choice may send to the two-pass path (their handles
// build the two-pass copy of U with the weights).
bool two_pass_possible(int C, int K) { return C <= 128 && K <= 256 && 2 * K >= C; }

// Two-pass instead of three-pass (automatic choice), from MI355X forwards
// (us, three-pass vs two-pass, warm / cache-cold): 128@28^2 B=24 26.7 / 32.7
// vs 22.4 / 31.2, B=32 27.8 / 35.3 vs 24.1 / 32.3, B=40 30.0 / 40.9 vs 26.8 /
// 36.8; 96@28^2 B=32 26.7 / 32.9 vs 20.2 / 28.0, B=48 32.5 / 40.6 vs 23.8 /
// 33.0; 72@28^2 B=32 25.4 / 30.5 vs 18.9 / 25.8; 64@56^2 B=8 21.5 / 26.4 vs
// 16.7 / 23.3; 128->64@28^2 B=32 24.1 / 31.4 vs 22.6 / 31.0; 48->40@13^2
// B=128 23.0 / 30.9 vs 17.3 / 23.0; 64->48@28^2 B=64 29.1 / 34.7 vs 21.5 /
// 28.4; 128@112^2 B=1 24.2 / 28.9 vs 20.7 / 29.4. It loses with
// few workgroups (128@28^2 B=4 12.3 vs 16.8, B=8 17.5 vs 19.7) and with a
// second round of them (128@28^2 B=64 36.7 vs 41.5; 128->256 B=32 34.9 vs
// 39.9). Channels-last the same (128@28^2 B=32 26.6 / 36.3 vs 23.7 / 31.5;
// 96@28^2 B=32 26.1 / 31.9 vs 19.1 / 26.8; 48->40@13^2 B=128 22.1 / 27.6 vs
// 16.8 / 22.0). Above 128 output channels the three-pass GEMM and output
// transform stay ahead on small grids (128->256@14^2 B=16, 72 workgroups: 18.2
// vs 20.0; 128->256@28^2 B=8, 104: 20.2 vs 21.2; 128->512@7^2 B=32: 21.4 vs
// 24.1) and fall behind from 128 workgroups on (128->256@14^2 B=32 23.7 / 30.6
// vs 21.0 / 27.9, B=48 29.1 vs 24.0; 128->256@28^2 B=12 24.2 vs 21.9, B=16
// 26.7 vs 22.4; 96->256@14^2 B=32 23.1 vs 16.8; 64->256@28^2 B=16 25.0 vs
// 16.8, B=20 28.2 vs 18.2; 128->192@14^2 B=48 26.1 vs 21.5): each two-pass
// workgroup reads all Cp channels of its operands, so its time follows Cp,
// not K. Grids of at most one 16-channel workgroup per CU run 16 output
// channels per workgroup, two per CU (gemm_out_kb); at most 64 input
// channels that admits grids of 64 such workgroups (64@56^2 B=4, 100
// workgroups: small-problem kernel 14.5 vs 12.8 us; B=8, 200: three-pass 18.5
// vs 13.8). With V and M written through the L2 (the three-pass path's two
// launch boundaries got cheaper) the three-pass path moved ahead at 128
// input channels below 128 such workgroups (128@28^2 B=8, 104: 15.49 vs
// 15.91) and above 128 output channels below three quarters of the CUs
// (128->256@14^2 B=32, 144: 20.49 vs 21.35; B=48, 216: 26.21 vs 24.14;
// 128->256@28^2 B=16, 200: 24.62 vs 23.43).
bool two_pass_wins(const Handle* Hd, const Shape& s) {
    if (!two_pass_possible(Hd->C, Hd->K)) return false;
    const int bp = (int)std::min<int64_t>(s.BP, INT32_MAX);
    const int64_t grid = gemm_out_grid(Hd->K, bp);
    const int64_t v_bytes = 2 * gemm_out_v_elems(Hd->Cp, s.BP);
    if (grid > Hd->cus || v_bytes > (int64_t)20 << 20) return false;
    if (Hd->K > 128) return 4 * grid >= 3 * (int64_t)Hd->cus;
    const int64_t min_grid = Hd->Cp > 64 ? 128 : 64;
    return gemm_out_grid(Hd->K, bp, gemm_out_kb(Hd->K, bp, Hd->cus)) >= min_grid;
}

bool in_gemm_plan_for(const Handle* Hd, const Shape& s, InGemmPlan* p) {
    const int64_t Bc = sub_batch(Hd, s);
    return in_gemm_plan((int)Bc, Hd->C, Hd->K, Hd->Cp, s.nh, s.nw, s.pad, Hd->cus, p);
}

// The input transform fused into the products (path 7) instead of the
// three-pass path's first two launches, for the GEMV-like shapes that the
// block GEMM serves (every sub-batch at most 32 tiles) with at most 128
// output channels. Every output-channel group of a position row repeats the
// row's transform, so the fused launch pays off only with few such groups;
// measured on MI355X (whole forwards, graph of ten, us, three-pass vs path
// 7): ResNet-50 conv3_x batch 1 9.28 vs 8.77, DenseNet-161 192 -> 48 at
// batch 1 28^2 9.49 vs 8.33, 14^2 8.91 vs 7.29, 7^2 8.65 vs 7.04; above 128
// output channels it loses (conv4_x 9.32 vs 9.98, conv5_x 11.72 vs 12.34 with
// the best plans).
bool in_gemm_wins(const Handle* Hd, const Shape& s) {
    InGemmPlan p;
    const int64_t BPc = sub_batch(Hd, s) * s.nh * s.nw;
    return Hd->K <= 128 && BPc <= 32 && in_gemm_plan_for(Hd, s, &p);
}

int choose_path(const Handle* Hd, const Shape& s) {
    if (Hd->path_pref == 1) return 1;
    if (Hd->path_pref == 4) return 4;
    if (Hd->path_pref == 6) return 6;
    if (Hd->path_pref == 7) {
        InGemmPlan p;
        return in_gemm_plan_for(Hd, s, &p) ? 7 : 1;
    }
    if (Hd->path_pref == 5) {
        FusedSmallPlan p;
        return fused_small_plan_for(Hd, s, &p) ? 5 : 1;
    }
    if (Hd->path_pref == 2) {
        if (Hd->nhwc) return 1;  // the position-row kernel reads and writes NCHW only
        FusedPlan p;
        return fused_plan_for(Hd, s, &p) ? 2 : 1;
    }
    if (Hd->path_pref == 3) {
        FusedBlockPlan p;
        return fused_block_plan_for(Hd, s, &p) ? 3 : 1;
    }
    // Automatic choice for layers with at most 64 input and output channels,
    // by a cost model fitted to MI355X forwards (36 shapes: C = K = 32 and 64
    // at 28^2-56^2, C = 48 -> K = 40 at 13^2, NCHW and NHWC, batch 2-192;
    // the rule picks the faster path in all but 5, which lose 0.2-3 us):
    //  * fused tile-block (its unstaged form, both layouts): its workgroups
    //    run one per CU, so the time steps by waves of workgroups over the
    //    CUs, ~3 us once + 9.2 us per 32-channel chunk and wave (conv2_x
    //    batch 16: 20.4 us, 32: 21.4, 128: 76.5; C = 32 batch 32: 12.5, 64:
    //    23.2; 64@112^2 batch 8: 21.2; channels-last conv2_x batch 16: 21.0,
    //    32: 21.9, 128: 78.6, C = 32 batch 32: 16.0);
    //  * three-pass: ~10 us of dependent launches plus its HBM bytes (x, y,
    //    V and M written and read) at 5 TB/s (conv2_x batch 16: 27.0 us,
    //    batch 128: 122 us).
    // Examples, three-pass vs fused (unstaged form), us: conv2_x B=8 21.1 vs
    // 20.6, B=16 27.4 vs 21.0, B=36 40.1 vs 23.4, B=40 41.6 vs 37.1; 64@28^2
    // B=64 29.3 vs 21.3; 32@56^2 B=8 18.7 vs 11.7, B=64 42.5 vs 23.3;
    // 64@112^2 B=8 33.4 vs 21.8, B=16 51.7 vs 41.5; 48->40@13^2 B=128 21.5
    // vs 19.5.
    // Small problems: one launch of the small-problem kernel while its grid
    // holds at most two workgroups per CU, four when the layer has two
    // 32-channel chunks (with one, the fused tile-block kernel is cheaper
    // there). Measured on MI355X, us, best other path vs small kernel:
    // conv2_x B=1 10.4 vs 6.8 (three-pass), B=3 14.2 vs 12.3, B=4 15.2 vs
    // 14.7 (two-pass), B=5 15.3 vs 15.5 (two-pass; 1000 workgroups);
    // 64@112^2 B=1 14.9 vs 13.3; 48@112^2 B=1 14.1 vs 12.4; 48->40@13^2 B=64
    // 15.1 vs 14.2; 32@56^2 B=4 11.0 vs 8.5, B=8 11.7 (fused tile-block) vs
    // 13.6; 32@112^2 B=2 11.7 vs 12.2; beyond four per CU it loses (64@112^2
    // B=2 16.2 vs 21.4; 48->40@13^2 B=128 16.9 vs 24.4). Where the two-pass
    // path can run, it takes over above two and a half small-problem
    // workgroups per CU (us, small kernel vs two-pass at 16 channels per
    // workgroup: 64@56^2 B=3, 2.3 per CU, 12.21 vs 12.62; B=4, 3.1: 14.51 vs
    // 12.80; B=5 15.14 vs 13.02; 64@28^2 B=16, 3.1: 13.71 vs 12.64; 48->40@13^2
    // B=64, 3.4: 14.01 vs 13.13; 48@56^2 B=4, 2.3: 11.88 vs 12.48).
    FusedSmallPlan sp;
    if (Hd->C <= 64 && Hd->K <= 64 && fused_small_plan_for(Hd, s, &sp)) {
        const int64_t cap2 = Hd->Cp <= 32 ? 4 : two_pass_wins(Hd, s) ? 5 : 8;  // 2 x per CU
        if (2 * sp.grid <= cap2 * (int64_t)Hd->cus) return 5;
    }
    FusedBlockPlan bp;
    if (Hd->C <= 64 && Hd->K <= 64 && fused_block_plan_for(Hd, s, &bp)) {
        const int64_t waves = (bp.grid + Hd->cus - 1) / Hd->cus;
        const int chunks = (Hd->Cp + 31) / 32;
        double t_fused = 3.0 + (double)waves * 9.2 * chunks;
        // with the short runs split off (fused_tail_first): the full runs'
        // rounds plus the small-problem launch (~6 us + 4 us per 2-tile
        // workgroup per CU, a 4-tile one counted twice: 11 us at 1.25 2-tile
        // workgroups per CU at 64@56^2 batch 40)
        Shape sb = s;
        sb.B = (int)sub_batch(Hd, s);
        FusedSmallPlan tp;
        const int tail = fused_tail_first(Hd, sb, bp, &tp);
        if (tail > 0) {
            const int64_t g_full = (int64_t)sb.B * (tail / 16) * bp.n_kblk;
            t_fused = 3.0 + (double)((g_full + Hd->cus - 1) / Hd->cus) * 9.2 * chunks + 6.0 +
                      2.0 * tp.tiles * (double)tp.grid / Hd->cus;
        }
        const double img = 2.0 * Hd->C * s.H * s.W + 2.0 * Hd->K * s.Ho * s.Wo +
                           4.0 * 64 * (Hd->Cp + Hd->K) * (double)s.nh * s.nw;
        const double t_three = 10.0 + s.B * img / 5.0e6;  // bytes / (5 TB/s) in us
        // The two-pass path beats the tile-block kernel from two 32-channel
        // chunks up while its grid leaves a fifth of the CUs free (us,
        // tile-block vs two-pass; NCHW, the unstaged form: 64@56^2 B=8 20.6
        // vs 16.3, B=12 20.8 vs 18.7, B=16 21.0 vs 20.0; 64@28^2 B=32 20.9 vs
        // 18.3, B=48 21.1 vs 19.1; 48@56^2 B=16 19.8 vs 17.7; 64->48@28^2
        // B=32 19.8 vs 18.0; 48->40@13^2 B=128 19.5 vs 17.1; 64@112^2 B=2
        // 20.5 vs 16.4, B=4 20.9 vs 20.2; NHWC, the staged form: 64@56^2
        // B=12 24.6 vs 19.0, B=16 25.0 vs 20.0; 64@28^2 B=48 24.0 vs 18.6);
        // not at one chunk (32@56^2 B=32 12.6 vs 18.6), nor from about 200
        // two-pass workgroups on, where the two trade places by shape
        // (64@28^2 B=64, 200: 21.3 vs 22.4; 64@224^2 B=1, 182: 20.9 vs 24.1;
        // 64@56^2 B=20, 250: 21.3 vs 23.1; 48->40@13^2 B=192, 216: 19.9 vs
        // 20.4).
        if (t_fused < t_three) {
            const int64_t grid = gemm_out_grid(Hd->K, (int)std::min<int64_t>(s.BP, INT32_MAX));
            const bool two = Hd->Cp > 32 && 5 * grid <= 4 * (int64_t)Hd->cus && two_pass_wins(Hd, s);
            return two ? 6 : 3;
        }
    }
    if (two_pass_wins(Hd, s)) return 6;
    return in_gemm_wins(Hd, s) ? 7 : 1;
}

// Core forward on one sub-batch. V/M are workspaces large enough for it.
// blocks: the GEMM on operand blocks (GEMV-like shapes, wgemm_blocks), V in
// the two-pass layout and U from the handle's block copy.
bool run_three_pass(Handle* Hd, const uint16_t* x, uint16_t* y, const Shape& s, uint16_t* V,
                    uint16_t* M, bool remember, const Epilogue& ep, bool timed = true,
                    bool blocks = false) {
    Profiler& pf = Hd->prof;
    const hipStream_t st = Hd->stream;
    const int C = Hd->C, K = Hd->K, Cp = Hd->Cp;
    const uint16_t* U = blocks ? Hd->Uw : Hd->U;
    const bool nhwc = Hd->nhwc != 0;
    // V streamed past the L2 (nt stores) when the GEMM reads it at most 4
    // times and it holds at most 24 MB; larger V are read faster from the L2
    // (whole forwards in a graph, us, streamed vs not: ResNet-50 batch 128
    // 128@28^2 (V 52 MB) 61.3 vs 58.1, 256@14^2 (38 MB) 52.1 vs 50.6, 512@7^2
    // (34 MB) 54.7 vs 50.9; batch 64 128@28^2 (26 MB) 37.5 vs 37.2; batch 32
    // 128@28^2 (13 MB) 27.1 vs 28.8, 256@14^2 (9 MB) 26.1 vs 27.1)
    const bool stream_v = !blocks && wgemm_v_reads(K, (int)s.BP) <= 4 &&
                          2 * (int64_t)64 * Cp * s.BP <= ((int64_t)24 << 20);
    const int vfrag = blocks ? (Cp + 31) / 32 : 0;
    const int64_t pstride = blocks ? gemm_out_v_elems(Cp, s.BP) / 64 : (int64_t)Cp * s.BP;
    auto in = [=]() {
        return launch_input_transform(x, V, s.B, C, s.H, s.W, s.pad, s.nh, s.nw, Cp, pstride, st,
                                      nhwc, stream_v, vfrag);
    };
    auto gm = [=]() {
        return blocks ? launch_wgemm_blocks(U, V, M, K, Cp, (int)s.BP, st)
                      : launch_wgemm(U, V, M, K, Cp, (int)s.BP, st);
    };
    auto out = [=]() {
        return launch_output_transform(M, y, s.B, K, s.Ho, s.Wo, s.nh, s.nw, K,
                                       (int64_t)K * s.BP, st, ep, nhwc);
    };
    if (remember) {
        pf.last[kKindInput] = in;
        pf.last[kKindGemm] = gm;
        pf.last[kKindOutput] = out;
        pf.last[kKindFused] = nullptr;
    }
    // timed = false (allocation-free forwards): never arm the profiler, whose
    // event pool may grow
    size_t e = timed ? pf.arm() : SIZE_MAX;
    const bool ok_in = hip_ok(in(), "input transform");
    pf.done(kKindInput, e, "input_transform_kernel");
    if (!ok_in) return false;
    e = timed ? pf.arm() : SIZE_MAX;
    const bool ok_gm = hip_ok(gm(), "wgemm");
    pf.done(kKindGemm, e, blocks ? wgemm_blocks_name((int)s.BP) : wgemm_name(K, Cp, (int)s.BP));
    if (!ok_gm) return false;
    e = timed ? pf.arm() : SIZE_MAX;
    const bool ok_out = hip_ok(out(), "output transform");
    pf.done(kKindOutput, e, "output_transform_kernel");
    return ok_out;
}

// Two-pass forward on one sub-batch (path 6): the three-pass input transform
// into V, then the products and the output transform in one launch (M stays
// on chip). Same V, M and y as run_three_pass, bit for bit.
bool run_two_pass(Handle* Hd, const uint16_t* x, uint16_t* y, const Shape& s, uint16_t* V,
                  bool remember, const Epilogue& ep) {
    Profiler& pf = Hd->prof;
    const hipStream_t st = Hd->stream;
    const int C = Hd->C, K = Hd->K, Cp = Hd->Cp;
    const uint16_t* U = Hd->Uw;
    const bool nhwc = Hd->nhwc != 0;
    // V in the two-pass block layout: the 16-byte pieces of a line come from
    // up to 8 workgroups, so V goes through the L2, where they merge (streamed
    // past it, the partial lines reach memory one by one: conv3_x batch 32,
    // cache-cold forward 35.9 -> 47.9 us)
    const bool stream_v = false;
    const int vfrag = (Cp + 31) / 32;
    const int64_t pstride = gemm_out_v_elems(Cp, s.BP) / 64;
    auto in = [=]() {
        return launch_input_transform(x, V, s.B, C, s.H, s.W, s.pad, s.nh, s.nw, Cp, pstride, st,
                                      nhwc, stream_v, vfrag);
    };
    const int go_kb = gemm_out_kb(K, (int)s.BP, Hd->cus);
    auto go = [=]() {
        return launch_gemm_out(U, V, y, s.B, K, Cp, s.nh, s.nw, s.Ho, s.Wo, st, ep, nhwc, go_kb);
    };
    if (remember) {
        pf.last[kKindInput] = in;
        pf.last[kKindGemm] = nullptr;
        pf.last[kKindOutput] = nullptr;
        pf.last[kKindFused] = go;
    }
    size_t e = pf.arm();
    const bool ok_in = hip_ok(in(), "input transform");
    pf.done(kKindInput, e, "input_transform_kernel");
    if (!ok_in) return false;
    e = pf.arm();
    const bool ok_go = hip_ok(go(), "products + output transform");
    pf.done(kKindFused, e, "gemm_out_kernel");
    return ok_go;
}

// Path 7 on one sub-batch: the input transform fused into the products (M
// to memory), then the three-pass output transform. Same M and y as
// run_three_pass, bit for bit.
bool run_in_gemm(Handle* Hd, const uint16_t* x, uint16_t* y, const Shape& s, uint16_t* M,
                 bool remember, const Epilogue& ep, bool timed) {
    Profiler& pf = Hd->prof;
    const hipStream_t st = Hd->stream;
    const int C = Hd->C, K = Hd->K, Cp = Hd->Cp;
    const uint16_t* U = Hd->Uw;
    const bool nhwc = Hd->nhwc != 0;
    InGemmPlan ip;
    if (!in_gemm_plan((int)s.B, C, K, Cp, s.nh, s.nw, s.pad, Hd->cus, &ip)) {
        set_error(kErrInvalidArgument, "no input-transform + products plan for this sub-batch");
        return false;
    }
    auto gm = [=]() {
        return launch_in_gemm(x, U, M, s.B, C, K, Cp, s.H, s.W, s.pad, s.nh, s.nw, ip, st, nhwc);
    };
    auto out = [=]() {
        return launch_output_transform(M, y, s.B, K, s.Ho, s.Wo, s.nh, s.nw, K,
                                       (int64_t)K * s.BP, st, ep, nhwc);
    };
    if (remember) {
        pf.last[kKindInput] = nullptr;
        pf.last[kKindGemm] = gm;
        pf.last[kKindOutput] = out;
        pf.last[kKindFused] = nullptr;
    }
    // timed = false (allocation-free forwards): never arm the profiler, whose
    // event pool may grow
    size_t e = timed ? pf.arm() : SIZE_MAX;
    const bool ok_gm = hip_ok(gm(), "input transform + products");
    pf.done(kKindGemm, e, in_gemm_name(ip));
    if (!ok_gm) return false;
    e = timed ? pf.arm() : SIZE_MAX;
    const bool ok_out = hip_ok(out(), "output transform");
    pf.done(kKindOutput, e, "output_transform_kernel");
    return ok_out;
}

// ---- scratch of the allocation-free forward (nova_forward_noalloc) -------
// The three-pass V/M workspace for callers that cannot allocate device
// memory. One copy per GPU, in device memory the loader reserves with the
// library's code object; it lives until the process ends. In host code the
// name `scratch` is only a stand-in symbol, never a device address: the
// kernels get the per-device address that hipGetSymbolAddress returns.
static __device__ __align__(256) unsigned char scratch[NOVA_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on device dev, looked up once per device with
// that device current (each GPU holds its own copy at its own address).
void* scratch_ptr(int dev, const char* fn) {
    if (dev < 0 || dev >= kMaxDevices) {
        set_error(kErrInvalidArgument, "%s: device %d out of range", fn, dev);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        int cur = 0;
        if (!hip_ok(hipGetDevice(&cur), "hipGetDevice")) return nullptr;
        if (cur != dev && !hip_ok(hipSetDevice(dev), "hipSetDevice")) return nullptr;
        void* p = nullptr;
        const bool ok = hip_ok(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                               "hipGetSymbolAddress(scratch)");
        if (cur != dev) (void)hipSetDevice(cur);
        if (!ok || p == nullptr) return nullptr;
        g_scratch_ptr[dev] = p;
    }
    return g_scratch_ptr[dev];
}

// Core forward. V_user/M_user may be null; caps are in fp16 elements.
// scratch_dev != null: the allocation-free form -- the three-pass workspace is
// that buffer (NOVA_NOALLOC_SCRATCH_BYTES), batches are split to fit it, and
// nothing is allocated (no workspace, counters, fragment copy or profiler
// events).
void forward_impl(Handle* Hd, const void* x, void* y, const Shape& s_all, void* V_user,
                  int64_t V_cap, void* M_user, int64_t M_cap, const char* fn,
                  void* scratch_dev = nullptr) {
    const bool no_alloc = scratch_dev != nullptr;
    if (!Hd->ready) {
        set_error(kErrNotInitialized, "%s: call nova_set_weights() before forward", fn);
        return;
    }
    if (s_all.B == 0) return;  // nothing to read or write (an empty tensor's pointer may be null)
    if (x == nullptr || y == nullptr) {
        set_error(kErrInvalidArgument, "%s: null input or output pointer", fn);
        return;
    }
    int64_t chunk = batch_chunk(Hd, s_all);
    if (chunk < 1) {
        set_error(kErrInvalidArgument, "%s: a single image of this shape exceeds 1 GB buffers", fn);
        return;
    }
    int path = choose_path(Hd, s_all);
    // the channels-last tile-block kernel stages x with 16-byte loads
    // (the staged channels-last form, above 64 channels, loads 16 bytes at a time)
    if (path == 3 && Hd->nhwc && Hd->Cp > 64 && !aligned16(x)) path = 1;
    if (path == 4) chunk = std::min(chunk, window_images(Hd, s_all));
    if (no_alloc) {
        // the position-row kernel needs an allocated M buffer and counters,
        // and a fragment copy not yet built would be allocated here
        if (path == 2 || path == 6 || ((path == 3 || path == 5) && !Hd->uf_ready) ||
            (path == 7 && (!Hd->uw_ready || 2 * (int64_t)64 * Hd->K * s_all.nh * s_all.nw >
                                                 (int64_t)NOVA_NOALLOC_SCRATCH_BYTES)))
            path = 1;
        const int64_t per_img = 2 * (int64_t)64 * (Hd->Cp + Hd->K) * s_all.nh * s_all.nw;
        if ((path == 1 || path == 4) && per_img > (int64_t)NOVA_NOALLOC_SCRATCH_BYTES - 256) {
            set_error(kErrWorkspace,
                      "%s: one image needs %lld bytes of workspace; the allocation-free "
                      "forward holds %lld",
                      fn, (long long)per_img, (long long)NOVA_NOALLOC_SCRATCH_BYTES);
            return;
        }
        // V, then M at the next 256-byte boundary (path 7: M only)
        if (path == 1 || path == 4)
            chunk = std::min<int64_t>(chunk, (NOVA_NOALLOC_SCRATCH_BYTES - 256) / per_img);
        if (path == 7)
            chunk = std::min<int64_t>(
                chunk, NOVA_NOALLOC_SCRATCH_BYTES / (2 * (int64_t)64 * Hd->K * s_all.nh * s_all.nw));
    }
    const bool fused = path == 2 || path == 3 || path == 5;
    if (fused && !ensure_uf(Hd)) return;
    if ((path == 6 || path == 7) && !ensure_uw(Hd)) return;
    if (path == 1 && (Hd->path_pref == 2 || Hd->path_pref == 3 || Hd->path_pref == 5 ||
                      Hd->path_pref == 7)) {
        set_error(kErrInvalidArgument, "%s: fused path unsupported for this shape; ran 3-pass", fn);
    }
    Hd->last_path = path;

    // workspace for the largest sub-batch
    const int64_t Bc = std::min<int64_t>(chunk, s_all.B);
    const int64_t BPc = Bc * s_all.nh * s_all.nw;
    // GEMV-like three-pass GEMMs (every sub-batch at most 32 tiles) read
    // operand blocks: U's block copy is built here once per weights, which
    // the allocation-free forward may not do
    const bool blocks = (path == 1 || path == 4) && !no_alloc &&
                        wgemm_blocks(Hd->K, Hd->Cp, (int)std::min<int64_t>(BPc, INT32_MAX));
    if (blocks && !ensure_uw(Hd)) return;
    const int64_t needV = path == 7 ? 0
                          : (path == 6 || blocks) ? gemm_out_v_elems(Hd->Cp, BPc)
                                                  : 64 * (int64_t)Hd->Cp * BPc;
    const int64_t needM = 64 * (int64_t)Hd->K * BPc;
    uint16_t* V = nullptr;
    uint16_t* M = nullptr;
    if (!fused && no_alloc) {
        V = static_cast<uint16_t*>(scratch_dev);
        M = V + ((needV + 127) & ~(int64_t)127);  // 256-byte aligned
    } else if (!fused) {
        size_t ws_bytes = 0;
        const bool userV = needV == 0 || (V_user && needV <= V_cap && aligned16(V_user));
        const bool userM = path == 6 || (M_user && needM <= M_cap && aligned16(M_user));
        if (!userV) ws_bytes += (size_t)needV * 2;
        if (!userM) ws_bytes += (size_t)needM * 2;
        if (ws_bytes && !ensure_ws(Hd, ws_bytes)) return;
        uint8_t* wsp = static_cast<uint8_t*>(Hd->ws);
        if (userV) {
            V = static_cast<uint16_t*>(V_user);
        } else {
            V = reinterpret_cast<uint16_t*>(wsp);
            wsp += (size_t)needV * 2;
        }
        M = path == 6 ? nullptr
                      : userM ? static_cast<uint16_t*>(M_user) : reinterpret_cast<uint16_t*>(wsp);
    }

    Profiler& pf = Hd->prof;
    const int64_t x_img = (int64_t)Hd->C * s_all.H * s_all.W;
    const int64_t y_img = (int64_t)Hd->K * s_all.Ho * s_all.Wo;
    for (int64_t b0 = 0; b0 < s_all.B; b0 += chunk) {
        Shape s = s_all;
        s.B = (int)std::min<int64_t>(chunk, s_all.B - b0);
        s.BP = (int64_t)s.B * s.nh * s.nw;
        const uint16_t* xx = static_cast<const uint16_t*>(x) + b0 * x_img;
        uint16_t* yy = static_cast<uint16_t*>(y) + b0 * y_img;
        Epilogue ep = Hd->ep;  // the residual follows the output's sub-batch
        if (ep.residual) ep.residual += b0 * y_img;
        if (path == 5) {
            const hipStream_t st = Hd->stream;
            const uint16_t* U = Hd->Uf;
            const int C = Hd->C, K = Hd->K, Cp = Hd->Cp;
            const bool nhwc = Hd->nhwc != 0;
            FusedSmallPlan sp;
            if (!fused_small_plan((int)s.B, C, K, Cp, s.nh, s.nw, Hd->cus, &sp)) {
                set_error(kErrInvalidArgument, "%s: no fused plan for this sub-batch", fn);
                return;
            }
            auto fz = [=]() {
                return launch_fused_small(xx, U, yy, s.B, C, K, Cp, s.H, s.W, s.pad, s.nh, s.nw,
                                          s.Ho, s.Wo, sp, st, ep, nhwc);
            };
            if (b0 == 0 && !no_alloc) {
                for (int k = 0; k < kNumKinds; k++) pf.last[k] = nullptr;
                pf.last[kKindFused] = fz;
            }
            const size_t e0 = no_alloc ? SIZE_MAX : pf.arm();
            const bool ok = hip_ok(fz(), "fused small kernel");
            pf.done(kKindFused, e0, "fused_small_kernel");
            if (!ok) return;
        } else if (path == 3) {
            const hipStream_t st = Hd->stream;
            const uint16_t* U = Hd->Uf;
            const int C = Hd->C, K = Hd->K, Cp = Hd->Cp;
            FusedBlockPlan bp;
            if (!fused_block_plan((int)s.B, C, K, Cp, s.H, s.W, s.nh, s.nw, &bp,
                                  Hd->nhwc != 0)) {
                set_error(kErrInvalidArgument, "%s: no fused plan for this sub-batch", fn);
                return;
            }
            // the short last run of every image to the small-problem kernel
            // when that saves the tile-block kernel a round of workgroups
            FusedSmallPlan sp{};
            const int tail = fused_tail_first(Hd, s, bp, &sp);
            if (tail > 0) {
                bp.nruns = tail / 16;
                bp.grid = (int64_t)s.B * bp.nruns * bp.n_kblk;
            }
            const bool nhwc = Hd->nhwc != 0;
            auto fz = [=]() {
                // a timed forward: one span from the tile-block kernel's start
                // to the tail launch's end
                const KernelEvents ev = kernel_events();
                if (tail > 0 && ev.start != nullptr) kernel_events() = KernelEvents{ev.start, nullptr};
                hipError_t e = launch_fused_block(xx, U, yy, s.B, C, K, Cp, s.H, s.W, s.pad,
                                                  s.nh, s.nw, s.Ho, s.Wo, bp, st, ep);
                if (e == hipSuccess && tail > 0) {
                    if (ev.start != nullptr) kernel_events() = KernelEvents{nullptr, ev.stop};
                    e = launch_fused_small(xx, U, yy, s.B, C, K, Cp, s.H, s.W, s.pad, s.nh, s.nw,
                                           s.Ho, s.Wo, sp, st, ep, nhwc);
                }
                return e;
            };
            if (b0 == 0 && !no_alloc) {
                for (int k = 0; k < kNumKinds; k++) pf.last[k] = nullptr;
                pf.last[kKindFused] = fz;
            }
            // with the tail launch the span covers both kernels, and its name
            // says so (per-kernel times and byte models can tell them apart)
            const size_t e0 = no_alloc ? SIZE_MAX : pf.arm();
            const bool ok = hip_ok(fz(), "fused block kernel");
            pf.done(kKindFused, e0,
                    tail > 0 ? "fused_block_kernel+fused_small_kernel" : "fused_block_kernel");
            if (!ok) return;
        } else if (path == 2) {
            const hipStream_t st = Hd->stream;
            const uint16_t* U = Hd->Uf;
            const int C = Hd->C, K = Hd->K, Cp = Hd->Cp;
            FusedPlan fp;
            if (!fused_plan((int)s.B, C, K, Cp, s.H, s.W, s.nh, s.nw, &fp)) {
                set_error(kErrInvalidArgument, "%s: no fused plan for this sub-batch", fn);
                return;
            }
            if (!ensure_ws(Hd, (size_t)fp.ms_bytes) || !ensure_cnt(Hd, (size_t)fp.cnt_count))
                return;
            uint16_t* Ms = static_cast<uint16_t*>(Hd->ws);
            unsigned* cnt = Hd->cnt;
            auto fz = [=]() {
                return launch_fused(xx, U, yy, Ms, cnt, s.B, C, K, Cp, s.H, s.W, s.pad, s.nh,
                                    s.nw, s.Ho, s.Wo, fp, st, ep);
            };
            if (b0 == 0) {
                for (int k = 0; k < kNumKinds; k++) pf.last[k] = nullptr;
                pf.last[kKindFused] = fz;
            }
            const size_t e0 = pf.arm();
            const bool ok = hip_ok(fz(), "fused kernel");
            pf.done(kKindFused, e0, fused_name(fp));
            if (!ok) return;
        } else if (path == 6) {
            if (!run_two_pass(Hd, xx, yy, s, V, b0 == 0, ep)) return;
        } else if (path == 7) {
            if (!run_in_gemm(Hd, xx, yy, s, M, b0 == 0 && !no_alloc, ep, !no_alloc)) return;
        } else if (!run_three_pass(Hd, xx, yy, s, V, M, b0 == 0 && !no_alloc, ep, !no_alloc,
                                   blocks)) {
            return;
        }
    }
}

}  // namespace
}  // namespace nova

using namespace nova;

extern "C" {

nova_handle_t nova_create(void) {
    Handle* H = new (std::nothrow) Handle();
    if (!H) set_error(kErrOutOfMemory, "nova_create: out of host memory");
    return H;
}

void nova_destroy(nova_handle_t h) {
    if (h == nullptr) return;
    Handle* H = as_handle(h, "nova_destroy");
    if (!H) return;
    if (H->U) hip_ok(hipFree(H->U), "hipFree(U)");
    if (H->Uf) hip_ok(hipFree(H->Uf), "hipFree(Uf)");
    if (H->Uw) hip_ok(hipFree(H->Uw), "hipFree(Uw)");
    if (H->ws) hip_ok(hipFree(H->ws), "hipFree(workspace)");
    if (H->cnt) hip_ok(hipFree(H->cnt), "hipFree(counters)");
    for (hipEvent_t e : H->prof.pool) (void)hipEventDestroy(e);
    if (H->order_ev) (void)hipEventDestroy(H->order_ev);
    H->magic = 0;
    delete H;
}

}  // extern "C"

namespace {

void set_weights_impl(nova_handle_t h, const void* d_weight, int K, int C, bool w_f16,
                      const char* fn) {
    Handle* H = as_handle(h, fn);
    if (!H) return;
    if (d_weight == nullptr || K < 1 || C < 1) {
        set_error(kErrInvalidArgument, "%s: bad arguments (w=%p K=%d C=%d)", fn, d_weight, K, C);
        return;
    }
    const int Cp = pad8(C);
    const size_t need = (size_t)64 * K * Cp * sizeof(uint16_t);
    // The GEMM kernels address U with 32-bit byte offsets through buffer
    // resources (position p's matrix starts at 2*p*K*Cp bytes): U must stay
    // below 2 GB. Checked before any device call, so an oversized layer is an
    // error, never a wrapped offset.
    if ((int64_t)need >= ((int64_t)1 << 31)) {
        set_error(kErrInvalidArgument,
                  "%s: K=%d x C=%d needs a %lld-byte transformed filter; the kernels address "
                  "at most 2^31 - 1 bytes of it",
                  fn, K, C, (long long)need);
        H->ready = false;
        return;
    }
    if (need > H->U_cap) {
        if (H->U) {
            if (!hip_ok(hipFree(H->U), "hipFree(U)")) return;
            H->U = nullptr;
            H->U_cap = 0;
        }
        if (!hip_ok(hipMalloc(&H->U, need), "hipMalloc(U)")) {
            H->ready = false;
            return;
        }
        H->U_cap = need;
    }
    H->uf_ready = false;
    H->uw_ready = false;
    H->K = K;
    H->C = C;
    H->Cp = Cp;
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) == hipSuccess) {
        H->device = dev;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) ==
                hipSuccess &&
            cus > 0)
            H->cus = cus;
    }
    H->ready = hip_ok(launch_filter_transform_gemm(d_weight, w_f16, H->U, K, C, Cp, H->stream),
                      "filter transform");
    const bool fused_possible = (C <= 64 && K <= 64 && H->path_pref == 0) ||
                                H->path_pref == 2 || H->path_pref == 3 || H->path_pref == 5;
    if (H->ready && fused_possible) H->ready = ensure_uf(H);
    if (H->ready && (H->path_pref == 6 || (H->path_pref == 0 && two_pass_possible(C, K))))
        H->ready = ensure_uw(H);
}

}  // namespace

extern "C" {

void nova_set_weights(nova_handle_t h, const void* d_weight, int K, int C) {
    set_weights_impl(h, d_weight, K, C, false, "nova_set_weights");
}

void nova_set_weights_f16(nova_handle_t h, const void* d_weight_f16, int K, int C) {
    set_weights_impl(h, d_weight_f16, K, C, true, "nova_set_weights_f16");
}

void nova_forward(nova_handle_t h, const void* d_input, void* d_output, int batch, int H,
                  int W, int pad) {
    Handle* Hd = as_handle(h, "nova_forward");
    if (!Hd) return;
    Shape s;
    if (!make_shape(Hd, batch, H, W, pad, &s, "nova_forward")) return;
    forward_impl(Hd, d_input, d_output, s, nullptr, 0, nullptr, 0, "nova_forward");
}

void nova_forward_noalloc(nova_handle_t h, const void* d_input, void* d_output, int batch, int H,
                          int W, int pad) {
    Handle* Hd = as_handle(h, "nova_forward_noalloc");
    if (!Hd) return;
    Shape s;
    if (!make_shape(Hd, batch, H, W, pad, &s, "nova_forward_noalloc")) return;
    if (!Hd->ready) {
        set_error(kErrNotInitialized, "nova_forward_noalloc: call nova_set_weights() before forward");
        return;
    }
    void* scr = scratch_ptr(Hd->device, "nova_forward_noalloc");
    if (scr == nullptr) return;
    forward_impl(Hd, d_input, d_output, s, nullptr, 0, nullptr, 0, "nova_forward_noalloc", scr);
}

void nova_forward_workspace(nova_handle_t h, const void* d_input, void* d_output,
                            void* d_V_gemm, void* d_M_gemm, int batch, int H, int W, int pad,
                            int nh, int nw) {
    Handle* Hd = as_handle(h, "nova_forward_workspace");
    if (!Hd) return;
    Shape s;
    if (!make_shape(Hd, batch, H, W, pad, &s, "nova_forward_workspace")) return;
    if (nh < s.nh || nw < s.nw) {
        set_error(kErrWorkspace,
                  "nova_forward_workspace: tiling %dx%d does not cover the %dx%d output", nh, nw,
                  s.Ho, s.Wo);
        return;
    }
    const int64_t bp_user = (int64_t)batch * nh * nw;
    forward_impl(Hd, d_input, d_output, s, d_V_gemm, 64 * (int64_t)Hd->C * bp_user, d_M_gemm,
                 64 * (int64_t)Hd->K * bp_user, "nova_forward_workspace");
}

void nova_weight_grad(nova_handle_t h, const void* d_input, const void* d_grad_output,
                      void* d_grad_weight, int batch, int C, int K, int H, int W, int pad,
                      int grad_f32) {
    Handle* Hd = as_handle(h, "nova_weight_grad");
    if (!Hd) return;
    if (d_grad_weight == nullptr || batch < 0 || C < 1 || K < 1 || H < 1 || W < 1 || pad < 0 ||
        (grad_f32 != 0 && grad_f32 != 1) || H + 2 * pad - 2 < 1 || W + 2 * pad - 2 < 1 ||
        (batch > 0 && (d_input == nullptr || d_grad_output == nullptr))) {
        set_error(kErrInvalidArgument, "nova_weight_grad: bad arguments");
        return;
    }
    int dev = 0, cus = 0;
    if (!hip_ok(hipGetDevice(&dev), "hipGetDevice")) return;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus < 1)
        cus = 256;
    const WgradPlan pl = wgrad_plan(batch, C, K, H, W, pad, cus);
    if (!pl.ok) {
        set_error(kErrInvalidArgument,
                  "nova_weight_grad: one image of this shape exceeds the kernels' 32-bit offsets");
        return;
    }
    if (!ensure_ws(Hd, (size_t)pl.ws_bytes)) return;
    hip_ok(launch_wgrad(static_cast<const uint16_t*>(d_input), d_grad_output, grad_f32 != 0,
                        static_cast<float*>(d_grad_weight), batch, C, K, H, W, pad, pl, Hd->ws,
                        Hd->stream),
           "weight gradient");
}

void nova_compute_tiling(int H, int W, int pad, int* nh, int* nw, int* H_out, int* W_out) {
    if (!nh || !nw || !H_out || !W_out) {
        set_error(kErrInvalidArgument, "nova_compute_tiling: null output pointer");
        return;
    }
    reference_tiling(H, W, pad, nh, nw, H_out, W_out);
}

void nova_filter_transform(const void* d_weight, void* d_U_gemm, int K, int C) {
    if (!d_weight || !d_U_gemm || K < 1 || C < 1) {
        set_error(kErrInvalidArgument, "nova_filter_transform: bad arguments");
        return;
    }
    if (!hip_ok(launch_filter_transform_ref(static_cast<const float*>(d_weight),
                                            static_cast<uint16_t*>(d_U_gemm), K, C, nullptr),
                "filter transform"))
        return;
    hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
}

void nova_input_transform(const void* d_input, void* d_V_gemm, int batch, int C, int H, int W,
                          int pad, int nh, int nw, int BP) {
    if (!d_input || !d_V_gemm || batch < 0 || C < 1 || H < 1 || W < 1 || pad < 0 || nh < 1 ||
        nw < 1 || (int64_t)BP < (int64_t)batch * nh * nw) {
        set_error(kErrInvalidArgument, "nova_input_transform: bad arguments");
        return;
    }
    if (batch == 0) return;
    if (nh > 65535 || (int64_t)batch * ((C + 63) / 64) > 65535 ||
        2 * (int64_t)batch * C * H * W >= ((int64_t)1 << 31) ||
        2 * 64 * (int64_t)C * BP >= ((int64_t)1 << 31)) {
        set_error(kErrInvalidArgument, "nova_input_transform: shape exceeds launch limits");
        return;
    }
    hip_ok(launch_input_transform(static_cast<const uint16_t*>(d_input),
                                  static_cast<uint16_t*>(d_V_gemm), batch, C, H, W, pad, nh, nw, C,
                                  (int64_t)C * BP, nullptr),
           "input transform");
}

void nova_output_transform(const void* d_M_gemm, void* d_output, int batch, int K, int H_out,
                           int W_out, int nh, int nw, int BP) {
    if (!d_M_gemm || !d_output || batch < 0 || K < 1 || H_out < 1 || W_out < 1 || nh < 1 ||
        nw < 1 || (int64_t)BP < (int64_t)batch * nh * nw) {
        set_error(kErrInvalidArgument, "nova_output_transform: bad arguments");
        return;
    }
    if (batch == 0) return;
    if (nh > 65535 || (int64_t)batch * ((K + 63) / 64) > 65535 ||
        2 * (int64_t)batch * K * H_out * W_out >= ((int64_t)1 << 31) ||
        2 * 64 * (int64_t)K * BP >= ((int64_t)1 << 31)) {
        set_error(kErrInvalidArgument, "nova_output_transform: shape exceeds launch limits");
        return;
    }
    hip_ok(launch_output_transform(static_cast<const uint16_t*>(d_M_gemm),
                                   static_cast<uint16_t*>(d_output), batch, K, H_out, W_out, nh,
                                   nw, K, (int64_t)K * BP, nullptr),
           "output transform");
}

int nova_get_K(nova_handle_t h) {
    Handle* H = as_handle(h, "nova_get_K");
    return H ? H->K : 0;
}

int nova_get_C(nova_handle_t h) {
    Handle* H = as_handle(h, "nova_get_C");
    return H ? H->C : 0;
}

void* nova_get_U_gemm(nova_handle_t h) {
    Handle* H = as_handle(h, "nova_get_U_gemm");
    return H ? H->U : nullptr;
}

nova_handle_t nova_fused_create(void) { return nova_create(); }
void nova_fused_destroy(nova_handle_t h) { nova_destroy(h); }
void nova_fused_set_weights(nova_handle_t h, const void* d_weight, int K, int C) {
    nova_set_weights(h, d_weight, K, C);
}
void nova_fused_forward(nova_handle_t h, const void* d_input, void* d_output, int batch, int H,
                        int W, int pad) {
    nova_forward(h, d_input, d_output, batch, H, W, pad);
}
void nova_fused_compute_tiling(int H, int W, int pad, int* nh, int* nw, int* H_out, int* W_out) {
    nova_compute_tiling(H, W, pad, nh, nw, H_out, W_out);
}

int nova_get_last_error(void) {
    const int e = g_err;
    g_err = 0;
    return e;
}

const char* nova_get_last_error_message(void) { return g_msg; }

void nova_set_stream(nova_handle_t h, void* stream) {
    Handle* H = as_handle(h, "nova_set_stream");
    if (!H) return;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (s == H->stream) return;
    // Work already queued on the old stream reads (and the filter transform
    // writes) the handle's U, its fragment copy, workspace and counters, which
    // the new stream's work reuses: the new stream waits for everything queued
    // on the old one so far. Skipped while either stream is being captured
    // into a graph (a capture may not wait on work outside it; graph capture
    // starts from a synchronized device).
    if (H->U != nullptr && !is_capturing(H->stream) && !is_capturing(s)) {
        if (H->order_ev == nullptr &&
            !hip_ok(hipEventCreateWithFlags(&H->order_ev, hipEventDisableTiming),
                    "nova_set_stream: hipEventCreateWithFlags"))
            return;
        if (!hip_ok(hipEventRecord(H->order_ev, H->stream), "nova_set_stream: hipEventRecord") ||
            !hip_ok(hipStreamWaitEvent(s, H->order_ev, 0), "nova_set_stream: hipStreamWaitEvent"))
            return;
    }
    H->stream = s;
}

void nova_set_path(nova_handle_t h, int path) {
    Handle* H = as_handle(h, "nova_set_path");
    if (!H) return;
    if (path < 0 || path > 7) {
        set_error(kErrInvalidArgument, "nova_set_path: path must be 0 to 7");
        return;
    }
    H->path_pref = path;
    if ((path == 2 || path == 3 || path == 5) && H->ready)
        ensure_uf(H);  // fused forced after the weights
    if ((path == 6 || path == 7) && H->ready) ensure_uw(H);
}

void nova_set_window_bytes(nova_handle_t h, long long bytes) {
    Handle* H = as_handle(h, "nova_set_window_bytes");
    if (!H) return;
    if (bytes < 0) {
        set_error(kErrInvalidArgument, "nova_set_window_bytes: bytes must be >= 0");
        return;
    }
    H->window_bytes = bytes == 0 ? kDefaultWindowBytes : (int64_t)bytes;
}

void nova_set_epilogue(nova_handle_t h, const void* d_bias_f16, int relu) {
    Handle* H = as_handle(h, "nova_set_epilogue");
    if (!H) return;
    if (relu != 0 && relu != 1) {
        set_error(kErrInvalidArgument, "nova_set_epilogue: relu must be 0 or 1");
        return;
    }
    H->ep.bias = static_cast<const uint16_t*>(d_bias_f16);
    H->ep.relu = relu;
}

void nova_set_layout(nova_handle_t h, int nhwc) {
    Handle* H = as_handle(h, "nova_set_layout");
    if (!H) return;
    if (nhwc != 0 && nhwc != 1) {
        set_error(kErrInvalidArgument, "nova_set_layout: nhwc must be 0 or 1");
        return;
    }
    H->nhwc = nhwc;
}

void nova_set_residual(nova_handle_t h, const void* d_residual_f16) {
    Handle* H = as_handle(h, "nova_set_residual");
    if (!H) return;
    H->ep.residual = static_cast<const uint16_t*>(d_residual_f16);
}

int nova_get_last_path(nova_handle_t h) {
    Handle* H = as_handle(h, "nova_get_last_path");
    return H ? H->last_path : 0;
}

long long nova_workspace_bytes(nova_handle_t h, int batch, int H, int W, int pad) {
    Handle* Hd = as_handle(h, "nova_workspace_bytes");
    if (!Hd) return -1;
    Shape s;
    if (!make_shape(Hd, batch, H, W, pad, &s, "nova_workspace_bytes")) return -1;
    const int path = Hd->ready ? choose_path(Hd, s) : 1;
    if (path == 2 || path == 3 || path == 5) return 0;
    int64_t chunk = std::max<int64_t>(1, batch_chunk(Hd, s));
    if (path == 4) chunk = std::min(chunk, window_images(Hd, s));
    const int64_t BPc = std::min<int64_t>(chunk, s.B) * s.nh * s.nw;
    if (path == 6) return (long long)(gemm_out_v_elems(Hd->Cp, BPc) * 2);  // V only
    if (path == 7) return (long long)(64 * (int64_t)Hd->K * BPc * 2);      // M only
    if (wgemm_blocks(Hd->K, Hd->Cp, (int)std::min<int64_t>(BPc, INT32_MAX)))  // V in blocks + M
        return (long long)((gemm_out_v_elems(Hd->Cp, BPc) + 64 * (int64_t)Hd->K * BPc) * 2);
    return (long long)(64 * ((int64_t)Hd->Cp + Hd->K) * BPc * 2);
}

void nova_profile_enable(nova_handle_t h, int enable) {
    Handle* H = as_handle(h, "nova_profile_enable");
    if (!H) return;
    Profiler& pf = H->prof;
    if (enable && pf.pool.empty() && !pf.grow()) {
        set_error(kErrHip, "nova_profile_enable: hipEventCreate failed");
        return;
    }
    pf.on = enable != 0;
    pf.next = 0;
    pf.spans.clear();
}

int nova_profile_read(nova_handle_t h, double* total_ms, long long* count) {
    Handle* H = as_handle(h, "nova_profile_read");
    if (!H || !total_ms || !count) return -1;
    Profiler& pf = H->prof;
    for (int k = 0; k < kNumKinds; k++) {
        total_ms[k] = 0.0;
        count[k] = 0;
    }
    if (pf.next > 0 && !hip_ok(hipEventSynchronize(pf.pool[pf.next - 1]), "hipEventSynchronize"))
        return -1;
    for (const Profiler::Span& sp : pf.spans) {
        float ms = 0.0f;
        if (!hip_ok(hipEventElapsedTime(&ms, pf.pool[sp.e0], pf.pool[sp.e1]), "hipEventElapsedTime"))
            return -1;
        total_ms[sp.kind] += ms;
        count[sp.kind] += 1;
    }
    const int n = (int)pf.spans.size();
    pf.next = 0;
    pf.spans.clear();
    return n;
}

double nova_profile_replay(nova_handle_t h, int kind, int reps) {
    Handle* H = as_handle(h, "nova_profile_replay");
    if (!H) return -1.0;
    if (kind < 0 || kind >= kNumKinds || reps < 1 || !H->prof.last[kind]) {
        set_error(kErrInvalidArgument, "nova_profile_replay: no recorded launch of kind %d", kind);
        return -1.0;
    }
    hipEvent_t e0, e1;
    if (!hip_ok(hipEventCreate(&e0), "hipEventCreate")) return -1.0;
    if (!hip_ok(hipEventCreate(&e1), "hipEventCreate")) {
        (void)hipEventDestroy(e0);
        return -1.0;
    }
    double ms_avg = -1.0;
    bool ok = hip_ok(hipEventRecord(e0, H->stream), "hipEventRecord");
    for (int r = 0; ok && r < reps; r++) ok = hip_ok(H->prof.last[kind](), "replay launch");
    ok = ok && hip_ok(hipEventRecord(e1, H->stream), "hipEventRecord") &&
         hip_ok(hipEventSynchronize(e1), "hipEventSynchronize");
    float ms = 0.0f;
    if (ok && hip_ok(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime")) ms_avg = ms / reps;
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return ms_avg;
}

const char* nova_profile_kernel_name(nova_handle_t h, int kind) {
    Handle* H = as_handle(h, "nova_profile_kernel_name");
    if (!H || kind < 0 || kind >= kNumKinds) return "";
    return H->prof.names[kind];
}

const char* nova_version(void) { return "nova-winograd-mi355x 0.1.0 (gfx950)"; }

}  // extern "C"
