// dg_halo.hip -- halo send/recv plan of one rank (extract_halo_info) for gfx950.
// C ABI in include/dynamis_graph.h.
//
// Reference: dynamis_state/src/csrc/graph/dist_graph_ops_kernels.cu:104-188 builds the
// plan with a boundary gather, two sorted `unique` calls over (peer * N + atom) keys, a
// global->local lookup and an index_fill for the interior mask.  Here nothing is sorted:
//
//   edge pass   one pass over the edges marks recv atoms (a byte per atom) and sets bit p
//               of a per-atom peer set for every send pair (p, d) (one u64 word per 64
//               peers; an atomic OR only when the bit is still clear);
//   count pass  a wave walks 256 consecutive atom ids and counts, per peer, the atoms of
//               each set -- hist[p][unit], peer-major;
//   scan        one exclusive scan over hist gives every (peer, unit) its output offset:
//               peer-major order = grouped by peer, ascending id inside a peer, which is
//               exactly the order of the reference's sorted unique keys;
//   write pass  the same walk ranks each atom inside its unit with a wave ballot per
//               peer bit and stores it.
// The peers present in a wave are visited through the OR of the wave's peer words, so a
// wave whose atoms have no remote neighbour costs one load and one reduction.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <string>

#include "../../include/dynamis_graph.h"
#include "dg_scan.hpp"

namespace dg {
dg_status fail(dg_status st, const std::string& msg);
}

namespace {
using namespace dg;

constexpr int kUnit = 256;           // atom ids per wave unit
constexpr int kWaves = 4;            // wave units per workgroup
constexpr int64_t kMaxWorld = 4096;  // LDS: kWaves * world_size int32 per workgroup

inline size_t al(size_t x) { return (x + 255) & ~(size_t)255; }
inline unsigned nblk(int64_t n, int b = 256) { return (unsigned)((n + b - 1) / b); }

enum : unsigned { kErrEdge = 1, kErrPid = 2, kErrOuter = 4 };

struct Layout {
    int64_t n, W, nw, nu;
    size_t o_hdr, o_smask, o_rflag, o_g2l, o_pid, o_hs, o_hr, o_os, o_or, o_part, total;
};

Layout layout(int64_t n, int64_t W)
{
    Layout L;
    L.n = n;
    L.W = W;
    L.nw = (W + 63) / 64;
    L.nu = (n + kUnit - 1) / kUnit;
    size_t o = 0;
    auto take = [&](size_t b) { size_t r = o; o = al(o + (b ? b : 1)); return r; };
    const size_t nh = (size_t)(W * L.nu);
    L.o_hdr = take(64);
    L.o_smask = take(8 * (size_t)n * L.nw);
    L.o_rflag = take((size_t)n);
    L.o_g2l = take(4 * (size_t)n);
    L.o_pid = take(2 * (size_t)n);
    // the send and receive histograms side by side, scanned as one array: the receive
    // offsets then carry the send total, which their readers subtract
    L.o_hs = take(4 * 2 * nh);
    L.o_hr = L.o_hs + 4 * nh;
    L.o_os = take(8 * (2 * nh + 1));
    L.o_or = L.o_os + 8 * nh;
    L.o_part = take(8 * (2 * nh / kScanTile + 2));
    L.total = o;
    return L;
}

struct Args {
    int64_t n, W, nw, nu, R, num_local;
    int pid_dt;
    const void* pid;
    unsigned long long* smask;
    uint8_t* rflag;
    int* g2l;
    uint16_t* pid16;  // pid narrowed to 16 bits (kMaxWorld <= 65535): the edge pass
                      // gathers it at random, and 2 B/atom stays in L2
};

__device__ __forceinline__ int64_t pid_at(const void* pid, int dt, int64_t a)
{
    return dt == DG_I32 ? (int64_t)((const int*)pid)[a] : ((const int64_t*)pid)[a];
}

__device__ __forceinline__ unsigned long long wave_or(unsigned long long x)
{
    unsigned lo = (unsigned)x, hi = (unsigned)(x >> 32);
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        lo |= __shfl_xor(lo, o, 64);
        hi |= __shfl_xor(hi, o, 64);
    }
    lo = __builtin_amdgcn_readfirstlane(lo);
    hi = __builtin_amdgcn_readfirstlane(hi);
    return ((unsigned long long)hi << 32) | lo;
}

// Peer-set word w of atom a: the send set (bits of the peers that need a) or the recv set
// (the single bit of a's owner if a is a recv atom).
template <int RECV>
__device__ __forceinline__ unsigned long long set_word(const Args& A, int64_t a, int w)
{
    if (RECV) {
        if (!A.rflag[a]) return 0ull;
        const int64_t p = A.pid16[a];
        return (p >> 6) == w ? 1ull << (p & 63) : 0ull;
    }
    return A.smask[a * A.nw + w];
}

__global__ void clear_kernel(Args A, unsigned* hdr)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t nsm = A.n * A.nw;
    if (i < nsm) A.smask[i] = 0ull;
    if (i < A.n) {
        A.rflag[i] = 0;
        A.g2l[i] = -1;
        const int64_t p = pid_at(A.pid, A.pid_dt, i);
        A.pid16[i] = (uint64_t)p < (uint64_t)A.W ? (uint16_t)p : (uint16_t)0xffff;
    }
    if (i < 16) hdr[i] = 0u;
}

__global__ void g2l_kernel(Args A, const int64_t* __restrict__ outer, unsigned* err)
{
    const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= A.num_local) return;
    const int64_t a = outer[j];
    if ((uint64_t)a >= (uint64_t)A.n) {
        atomicOr(err, (unsigned)kErrOuter);
        return;
    }
    A.g2l[a] = (int)j;
}

// dist_graph_ops_kernels.cu:46-58 (boundary_peer_kernel) fused with the recv / send
// marking that the reference does with unique().  A thread takes kEdgeIlp consecutive
// edges, so that many pid gathers are in flight.  Edges of one dst arrive together, so a
// (dst, peer) pair usually repeats on neighbouring edges: only the first edge of a run of
// equal pairs (compared with the previous edge, across lanes too) touches the peer word.
constexpr int kEdgeIlp = 4;

__global__ __launch_bounds__(256) void edge_kernel(Args A, const int64_t* __restrict__ src,
                                                   const int64_t* __restrict__ dst, int64_t E,
                                                   unsigned* err)
{
    const int64_t e0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * kEdgeIlp;
    int64_t s[kEdgeIlp], d[kEdgeIlp], p[kEdgeIlp];
    bool ok[kEdgeIlp];
#pragma unroll
    for (int k = 0; k < kEdgeIlp; ++k) {
        const bool in = e0 + k < E;
        s[k] = in ? src[e0 + k] : 0;
        d[k] = in ? dst[e0 + k] : -1;
        ok[k] = in && (uint64_t)s[k] < (uint64_t)A.n && (uint64_t)d[k] < (uint64_t)A.n;
        if (in && !ok[k]) atomicOr(err, (unsigned)kErrEdge);
    }
#pragma unroll
    for (int k = 0; k < kEdgeIlp; ++k) {
        p[k] = ok[k] ? (int64_t)A.pid16[s[k]] : A.R;
        if ((uint64_t)p[k] >= (uint64_t)A.W) {
            atomicOr(err, (unsigned)kErrPid);
            ok[k] = false;
            p[k] = A.R;
        }
    }
    // pair key of each edge (-1: nothing to mark); the previous lane's last key
    int64_t key[kEdgeIlp];
#pragma unroll
    for (int k = 0; k < kEdgeIlp; ++k) key[k] = (ok[k] && p[k] != A.R) ? d[k] * A.W + p[k] : -1;
    const unsigned lo = __shfl_up((unsigned)key[kEdgeIlp - 1], 1, 64);
    const unsigned hi = __shfl_up((unsigned)((uint64_t)key[kEdgeIlp - 1] >> 32), 1, 64);
    int64_t prev = (threadIdx.x & 63) ? (int64_t)(((uint64_t)hi << 32) | lo) : -1;
#pragma unroll
    for (int k = 0; k < kEdgeIlp; ++k) {
        if (key[k] >= 0) {
            A.rflag[s[k]] = 1;
            if (key[k] != prev) {
                unsigned long long* wp = A.smask + d[k] * A.nw + (p[k] >> 6);
                const unsigned long long bit = 1ull << (p[k] & 63);
                if (!(__atomic_load_n(wp, __ATOMIC_RELAXED) & bit)) atomicOr(wp, bit);
            }
        }
        prev = key[k];
    }
}

// dist_graph_ops_kernels.cu:178-182: interior = no remote-src edge into the atom.
__global__ void interior_kernel(Args A, const int64_t* __restrict__ outer, uint8_t* __restrict__ mask)
{
    const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= A.num_local) return;
    const int64_t a = outer[j];
    uint8_t in = 1;
    if ((uint64_t)a < (uint64_t)A.n)
        for (int w = 0; w < A.nw; ++w)
            if (A.smask[a * A.nw + w]) in = 0;
    mask[j] = in;
}

// MODE 0: count per (peer, unit) into hist.  MODE 1: write, ranks from off.
template <int RECV, int MODE>
__global__ __launch_bounds__(256) void walk_kernel(Args A, int* __restrict__ hist,
                                                   const int64_t* __restrict__ off,
                                                   int64_t* __restrict__ out0,
                                                   int64_t* __restrict__ out1)
{
    extern __shared__ int s_run[];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    int* run = s_run + wv * A.W;
    const int64_t u = (int64_t)blockIdx.x * kWaves + wv;
    if (u >= A.nu) return;  // whole wave; no workgroup barrier below
    for (int p = lane; p < A.W; p += 64) run[p] = 0;
    const unsigned long long lt = (1ull << lane) - 1ull;
    // the receive offsets come from one scan with the send histogram in front, so they
    // carry the send total, which is their first entry
    const int64_t base = MODE == 1 && RECV ? off[0] : 0;
    const int64_t a0 = u * kUnit;
    for (int st = 0; st < kUnit && a0 + st < A.n; st += 64) {
        const int64_t a = a0 + st + lane;
        const bool ok = a < A.n;
        for (int w = 0; w < A.nw; ++w) {
            const unsigned long long m = ok ? set_word<RECV>(A, a, w) : 0ull;
            unsigned long long un = wave_or(m);
            while (un) {
                const int b = __builtin_ctzll(un);
                un &= un - 1;
                const int p = w * 64 + b;
                const bool has = (m >> b) & 1ull;
                const unsigned long long bal = __ballot(has);
                const int c = __popcll(bal);
                const int r = run[p];
                if (MODE == 1 && has) {
                    const int64_t pos = off[(int64_t)p * A.nu + u] - base + r + __popcll(bal & lt);
                    if (RECV) {
                        out0[pos] = a;                  // recv_atom_global
                        out1[pos] = A.num_local + pos;  // recv_ghost_indices
                    } else {
                        out0[pos] = (int64_t)A.g2l[a];  // send_local_indices
                    }
                }
                if (lane == 0) run[p] = r + c;
            }
        }
    }
    if (MODE == 0)
        for (int p = lane; p < A.W; p += 64) hist[(int64_t)p * A.nu + u] = run[p];
}

__global__ void offsets_kernel(const int64_t* __restrict__ os, const int64_t* __restrict__ orr,
                               int64_t W, int64_t nu, int64_t* __restrict__ send_off,
                               int64_t* __restrict__ recv_off, int64_t* __restrict__ tot)
{
    const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p > W) return;
    // (orr follows os in one scan: its entries carry the send total, orr[0])
    send_off[p] = os[p * nu];
    recv_off[p] = orr[p * nu] - orr[0];
    if (p == W) {
        tot[0] = os[W * nu];
        tot[1] = orr[W * nu] - orr[0];
    }
}

dg_status launch_ok(const char* what)
{
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(DG_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
    return DG_OK;
}

dg_status check_desc(const dg_halo_desc* d)
{
    if (!d) return fail(DG_ERR_INVALID, "desc is NULL");
    if (d->n_atoms < 0 || d->n_atoms >= (1LL << 31))
        return fail(DG_ERR_INVALID, "n_atoms must be in [0, 2^31)");
    if (d->n_edges < 0) return fail(DG_ERR_INVALID, "n_edges must be >= 0");
    if (d->num_local < 0 || d->num_local >= (1LL << 31))
        return fail(DG_ERR_INVALID, "num_local must be in [0, 2^31)");
    if (d->world_size < 1) return fail(DG_ERR_INVALID, "world_size must be >= 1, got " + std::to_string(d->world_size));
    if (d->world_size > kMaxWorld)
        return fail(DG_ERR_INVALID, "world_size must be <= 4096, got " + std::to_string(d->world_size));
    if (d->my_rank < 0 || d->my_rank >= d->world_size)
        return fail(DG_ERR_INVALID, "my_rank must be in [0, world_size)");
    if (d->pid_dtype != DG_I32 && d->pid_dtype != DG_I64)
        return fail(DG_ERR_INVALID, "pid must be int32 or int64");
    return DG_OK;
}

Args make_args(const dg_halo_desc* d, const Layout& L, const void* pid, void* ws)
{
    char* w = (char*)ws;
    Args A;
    A.n = L.n;
    A.W = L.W;
    A.nw = L.nw;
    A.nu = L.nu;
    A.R = d->my_rank;
    A.num_local = d->num_local;
    A.pid_dt = d->pid_dtype;
    A.pid = pid;
    A.smask = (unsigned long long*)(w + L.o_smask);
    A.rflag = (uint8_t*)(w + L.o_rflag);
    A.g2l = (int*)(w + L.o_g2l);
    A.pid16 = (uint16_t*)(w + L.o_pid);
    return A;
}

unsigned walk_grid(const Layout& L) { return (unsigned)((L.nu + kWaves - 1) / kWaves); }
size_t walk_lds(const Layout& L) { return (size_t)kWaves * L.W * sizeof(int); }

}  // namespace

extern "C" {

size_t dg_halo_workspace_size(int64_t n_atoms, int64_t world_size)
{
    if (n_atoms < 0 || world_size < 1 || world_size > kMaxWorld) return 0;
    return layout(n_atoms, world_size).total;
}

dg_status dg_halo_count(const dg_halo_desc* d, const int64_t* src, const int64_t* dst,
                        const void* pid, const int64_t* my_outer, int64_t* send_offsets,
                        int64_t* recv_offsets, uint8_t* interior_mask, void* ws, size_t ws_bytes,
                        hipStream_t s)
{
    dg_status st = check_desc(d);
    if (st != DG_OK) return st;
    Layout L = layout(d->n_atoms, d->world_size);
    if (ws_bytes < L.total) return fail(DG_ERR_WORKSPACE, "workspace too small");
    Args A = make_args(d, L, pid, ws);
    char* w = (char*)ws;
    unsigned* hdr = (unsigned*)(w + L.o_hdr);
    int64_t* tot = (int64_t*)hdr;   // [0] send total, [1] recv total
    unsigned* err = hdr + 4;
    const int64_t nclear = std::max<int64_t>(L.n * L.nw, std::max<int64_t>(L.n, 16));
    hipLaunchKernelGGL(clear_kernel, dim3(nblk(nclear)), dim3(256), 0, s, A, hdr);
    if (d->num_local > 0)
        hipLaunchKernelGGL(g2l_kernel, dim3(nblk(d->num_local)), dim3(256), 0, s, A, my_outer, err);
    if (d->n_edges > 0)
        hipLaunchKernelGGL(edge_kernel, dim3(nblk((d->n_edges + kEdgeIlp - 1) / kEdgeIlp)), dim3(256), 0, s, A, src, dst,
                           d->n_edges, err);
    if (d->num_local > 0)
        hipLaunchKernelGGL(interior_kernel, dim3(nblk(d->num_local)), dim3(256), 0, s, A, my_outer,
                           interior_mask);
    int* hs = (int*)(w + L.o_hs);
    int* hr = (int*)(w + L.o_hr);
    int64_t* os = (int64_t*)(w + L.o_os);
    int64_t* orr = (int64_t*)(w + L.o_or);
    int64_t* part = (int64_t*)(w + L.o_part);
    if (L.nu > 0) {
        hipLaunchKernelGGL((walk_kernel<0, 0>), dim3(walk_grid(L)), dim3(256), walk_lds(L), s, A, hs,
                           (const int64_t*)nullptr, (int64_t*)nullptr, (int64_t*)nullptr);
        hipLaunchKernelGGL((walk_kernel<1, 0>), dim3(walk_grid(L)), dim3(256), walk_lds(L), s, A, hr,
                           (const int64_t*)nullptr, (int64_t*)nullptr, (int64_t*)nullptr);
    }
    const int64_t nh = L.W * L.nu;
    device_excl_scan<int, int64_t>(hs, 2 * nh, os, part, s);  // hs, hr side by side
    hipLaunchKernelGGL(offsets_kernel, dim3(nblk(L.W + 1)), dim3(256), 0, s, (const int64_t*)os,
                       (const int64_t*)orr, L.W, L.nu, send_offsets, recv_offsets, tot);
    return launch_ok("dg_halo_count");
}

dg_status dg_halo_read_totals(const void* ws, int64_t* total_send, int64_t* total_recv,
                              hipStream_t s)
{
    int64_t h[3];
    hipError_t e = hipMemcpyAsync(h, ws, sizeof h, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess)
        return fail(DG_ERR_HIP, std::string("dg_halo_read_totals: ") + hipGetErrorString(e));
    if (total_send) *total_send = h[0];
    if (total_recv) *total_recv = h[1];
    const unsigned err = (unsigned)h[2];
    if (err & kErrEdge) return fail(DG_ERR_RANGE, "edge index out of range [0, N)");
    if (err & kErrPid) return fail(DG_ERR_RANGE, "pid_outer value out of range [0, world_size)");
    if (err & kErrOuter) return fail(DG_ERR_RANGE, "my_outer_atoms entry out of range [0, N)");
    return DG_OK;
}

dg_status dg_halo_write(const dg_halo_desc* d, const void* pid, int64_t* send_local_indices,
                        int64_t* recv_ghost_indices, int64_t* recv_atom_global, void* ws,
                        size_t ws_bytes, hipStream_t s)
{
    dg_status st = check_desc(d);
    if (st != DG_OK) return st;
    Layout L = layout(d->n_atoms, d->world_size);
    if (ws_bytes < L.total) return fail(DG_ERR_WORKSPACE, "workspace too small");
    if (L.nu == 0) return DG_OK;
    Args A = make_args(d, L, pid, ws);
    char* w = (char*)ws;
    const int64_t* os = (const int64_t*)(w + L.o_os);
    const int64_t* orr = (const int64_t*)(w + L.o_or);
    hipLaunchKernelGGL((walk_kernel<0, 1>), dim3(walk_grid(L)), dim3(256), walk_lds(L), s, A,
                       (int*)nullptr, os, send_local_indices, (int64_t*)nullptr);
    hipLaunchKernelGGL((walk_kernel<1, 1>), dim3(walk_grid(L)), dim3(256), walk_lds(L), s, A,
                       (int*)nullptr, orr, recv_atom_global, recv_ghost_indices);
    return launch_ok("dg_halo_write");
}

}  // extern "C"
