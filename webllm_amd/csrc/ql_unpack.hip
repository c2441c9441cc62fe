// Load-time unpack: GPTQ int4 -> fp16 [N, K] row-major, bit-identical to the reference loader's
// f32ToF16Bits(dequantizeGptqInt4(...)) (src/weights/quant.ts:42-118, src/gpu/buffer.ts:57-100).
//
// HBM-bound (read K*N/2 + scales/zeros, write 2*K*N bytes). The fast kernel reads a 16-packed-row
// x 64-column tile of qweight with 16-byte loads along N (the GPTQ layout is contiguous along N),
// dequantizes in packed fp16, transposes through LDS and writes 256 contiguous bytes per output
// row segment with streaming (nontemporal) stores: the fp16 arena is written once and not read
// back by this launch, and streaming stores measured 164 against 208 us for the 0.5B weight set.
// The generic kernel covers any K, N and alignment, one packed word per lane.
#include "ql_device.h"
#include "ql_internal.h"

namespace ql {

namespace {

typedef uint32_t v4u __attribute__((ext_vector_type(4)));
constexpr int kTileRows = 16;  // packed rows (128 k)

// one 16-byte chunk of the fp16 arena, written without allocating in the caches
__device__ __forceinline__ void store_stream(uint16_t* p, uint4 v)
{
    __builtin_nontemporal_store(__builtin_bit_cast(v4u, v), reinterpret_cast<v4u*>(p));
}
constexpr int kTileCols = 64;  // output rows n
constexpr int kPad = 17;       // LDS row pitch in 16-byte chunks (16 + 1 against bank conflicts)

__global__ __launch_bounds__(256) void unpack_tile_kernel(UnpackArgs a)
{
    __shared__ uint4 tile[kTileCols * kPad];
    const int t = threadIdx.x;
    const int n0 = blockIdx.x * kTileCols;
    const int p0 = blockIdx.y * kTileRows;
    const int P = a.K >> 3;               // K % 8 == 0 on this path
    const int NC = (a.N + 7) >> 3;

    const int r = t >> 4;                 // packed row within tile
    const int cq = t & 15;                // column quad
    const int p = p0 + r;
    const int n = n0 + 4 * cq;
    if (p < P && n < a.N) {               // N % 4 == 0: the whole quad is in range
        const uint4 w = *reinterpret_cast<const uint4*>(a.qweight + (size_t)p * a.N + n);
        const int g = (p * 8) / a.group;
        const uint2 sv = *reinterpret_cast<const uint2*>(a.scales + (size_t)g * a.N + n);
        uint32_t z[4];
        if (a.qzeros) {
            const uint32_t zw = a.qzeros[(size_t)g * NC + (n >> 3)] >> (4 * (n & 7));
#pragma unroll
            for (int u = 0; u < 4; u++) z[u] = ((zw >> (4 * u)) & 15u) + 1u;
        } else {
#pragma unroll
            for (int u = 0; u < 4; u++) z[u] = 8u;
        }
        const uint32_t words[4] = {w.x, w.y, w.z, w.w};
        const uint32_t s2[4] = {(sv.x & 0xffffu) * 0x10001u, (sv.x >> 16) * 0x10001u,
                                (sv.y & 0xffffu) * 0x10001u, (sv.y >> 16) * 0x10001u};
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const f16x8 h = dequant_word_natural(words[u], zero_pair(z[u]), s2[u]);
            tile[(4 * cq + u) * kPad + r] = __builtin_bit_cast(uint4, h);
        }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int c = t + 256 * i;        // chunk: column c/16, packed row c%16
        const int col = c >> 4;
        const int rr = c & 15;
        const int nn = n0 + col;
        const int pp = p0 + rr;
        if (nn < a.N && pp < P) store_stream(static_cast<uint16_t*>(a.out) + (size_t)nn * a.K + (size_t)pp * 8, tile[col * kPad + rr]);
    }
}

// Many tensors in one launch (the loader's whole weight set): the same 16 x 64 tiles, numbered
// across the batch; each workgroup walks tiles blockIdx.x, blockIdx.x + gridDim.x, ... and issues
// the next tile's loads before it transposes the current one through LDS, so every workgroup keeps
// two tiles of packed words in flight. Every tensor here meets the tile path's conditions.
struct TileLoad {
    uint4 w;
    uint2 sv;
    uint32_t zw;
    bool live;
};

__device__ __forceinline__ int batch_item(const UnpackBatch& b, int tile)
{
    int lo = 0, hi = b.count - 1;          // last item whose first tile is <= tile
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (b.it[mid].tile_begin <= tile) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

__device__ __forceinline__ TileLoad load_tile(const UnpackItem& it, int local, int r, int cq)
{
    const int tiles_n = (it.N + kTileCols - 1) / kTileCols;
    const int tp = local / tiles_n;
    const int p = tp * kTileRows + r;
    const int n = (local - tp * tiles_n) * kTileCols + 4 * cq;
    TileLoad l;
    l.live = p < (it.K >> 3) && n < it.N;
    l.w = uint4{0u, 0u, 0u, 0u};
    l.sv = uint2{0u, 0u};
    l.zw = 0x77777777u;                    // stored 7: zero 8 (no qzeros)
    if (l.live) {
        const int g = (p * 8) / it.group;
        l.w = *reinterpret_cast<const uint4*>(it.qweight + (size_t)p * it.N + n);
        l.sv = *reinterpret_cast<const uint2*>(it.scales + (size_t)g * it.N + n);
        if (it.qzeros) l.zw = it.qzeros[(size_t)g * ((it.N + 7) >> 3) + (n >> 3)];
        l.zw >>= 4 * (n & 7);
    }
    return l;
}

__global__ __launch_bounds__(256) void unpack_batch_kernel(const UnpackBatch b)
{
    __shared__ uint4 tile[kTileCols * kPad];
    const int t = threadIdx.x;
    const int r = t >> 4;                  // packed row within tile
    const int cq = t & 15;                 // column quad
    int cur = blockIdx.x;
    if (cur >= b.tiles) return;
    int ci = batch_item(b, cur);
    TileLoad l = load_tile(b.it[ci], cur - b.it[ci].tile_begin, r, cq);
    for (;;) {
        const int nxt = cur + (int)gridDim.x;
        const int ni = nxt < b.tiles ? batch_item(b, nxt) : ci;
        TileLoad ln{};
        if (nxt < b.tiles) ln = load_tile(b.it[ni], nxt - b.it[ni].tile_begin, r, cq);

        const UnpackItem& it = b.it[ci];
        const int local = cur - it.tile_begin;
        const int tiles_n = (it.N + kTileCols - 1) / kTileCols;
        const int tp = local / tiles_n;
        const int n0 = (local - tp * tiles_n) * kTileCols;
        const int p0 = tp * kTileRows;
        const int P = it.K >> 3;
        if (l.live) {
            const uint32_t words[4] = {l.w.x, l.w.y, l.w.z, l.w.w};
            const uint32_t s2[4] = {(l.sv.x & 0xffffu) * 0x10001u, (l.sv.x >> 16) * 0x10001u,
                                    (l.sv.y & 0xffffu) * 0x10001u, (l.sv.y >> 16) * 0x10001u};
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const f16x8 h = dequant_word_natural(words[u], zero_pair(((l.zw >> (4 * u)) & 15u) + 1u), s2[u]);
                tile[(4 * cq + u) * kPad + r] = __builtin_bit_cast(uint4, h);
            }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = t + 256 * i;     // chunk: column c/16, packed row c%16
            const int col = c >> 4;
            const int rr = c & 15;
            const int nn = n0 + col;
            const int pp = p0 + rr;
            if (nn < it.N && pp < P) store_stream(it.out + (size_t)nn * it.K + (size_t)pp * 8, tile[col * kPad + rr]);
        }
        if (nxt >= b.tiles) break;
        __syncthreads();                   // the tile is read before the next one overwrites it
        cur = nxt;
        ci = ni;
        l = ln;
    }
}

// fp32 [N, K]: exactly dequantizeGptqInt4 (quant.ts:112, (q - zero) * scale with the scale
// decoded from fp16; the product is exact in fp32). One packed word per lane, 2 x 16-byte stores
// when the row allows it.
__global__ __launch_bounds__(256) void unpack_f32_kernel(UnpackArgs a)
{
    const int n = blockIdx.x * 256 + threadIdx.x;
    const int p = blockIdx.y;
    if (n >= a.N) return;
    const int NC = (a.N + 7) >> 3;
    const int g = (p * 8) / a.group;
    const uint32_t w = a.qweight[(size_t)p * a.N + n];
    const int z = (int)zero_of(a.qzeros, g, NC, n);
    // (q - z) * s: one fp32 rounding of the exact product, as the reference's JS-number product
    // stored into a Float32Array (quant.ts:111-112); exact for fp16 scales
    const float s = a.scales_f32 ? a.scales_f32[(size_t)g * a.N + n]
                                 : (float)__builtin_bit_cast(_Float16, a.scales[(size_t)g * a.N + n]);
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; k++) v[k] = (float)((int)((w >> (4 * k)) & 15u) - z) * s;
    float* row = reinterpret_cast<float*>(a.out) + (size_t)n * a.K + (size_t)p * 8;
    if (a.K % 4 == 0 && (p + 1) * 8 <= a.K) {
        reinterpret_cast<float4*>(row)[0] = float4{v[0], v[1], v[2], v[3]};
        reinterpret_cast<float4*>(row)[1] = float4{v[4], v[5], v[6], v[7]};
    } else {
        for (int k = 0; k < 8 && p * 8 + k < a.K; k++) row[k] = v[k];
    }
}

// Any shape: lane = one packed word (p, n); up to 8 fp16 stores with the reference's K tail.
__global__ __launch_bounds__(256) void unpack_generic_kernel(UnpackArgs a)
{
    const int n = blockIdx.x * 256 + threadIdx.x;
    const int p = blockIdx.y;
    if (n >= a.N) return;
    const int NC = (a.N + 7) >> 3;
    const int g = (p * 8) / a.group;
    const uint32_t w = a.qweight[(size_t)p * a.N + n];
    const uint32_t z = zero_of(a.qzeros, g, NC, n);
    const _Float16 s = __builtin_bit_cast(_Float16, a.scales[(size_t)g * a.N + n]);
    const float sf = (float)s;
    for (int k = 0; k < 8; k++) {
        const int i = p * 8 + k;
        if (i >= a.K) break;
        const int q = (int)((w >> (4 * k)) & 15u);
        // (q - z) * s is exact in fp32 (at most 16 significant bits); one RNE rounding to fp16.
        const _Float16 h = (_Float16)((float)(q - (int)z) * sf);
        static_cast<uint16_t*>(a.out)[(size_t)n * a.K + i] = __builtin_bit_cast(uint16_t, h);
    }
}

}  // namespace

hipError_t launch_unpack_batch(const UnpackBatch& b, hipStream_t stream)
{
    // resident workgroups: 8 per CU (17 KB of LDS and 4 waves each), fewer for small batches
    const int grid = b.tiles < kPlanCUs * 8 ? b.tiles : kPlanCUs * 8;
    if (grid <= 0) return hipSuccess;
    hipLaunchKernelGGL(unpack_batch_kernel, dim3(grid), dim3(256), 0, stream, b);
    return hipGetLastError();
}

int unpack_tiles(int N, int K) { return ((N + kTileCols - 1) / kTileCols) * (((K >> 3) + kTileRows - 1) / kTileRows); }

hipError_t launch_unpack_f32(const UnpackArgs& a, hipStream_t stream)
{
    dim3 grid((a.N + 255) / 256, (a.K + 7) / 8);
    hipLaunchKernelGGL(unpack_f32_kernel, grid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_unpack(const UnpackArgs& a, bool fast, hipStream_t stream)
{
    const int P = (a.K + 7) / 8;
    if (fast) {
        dim3 grid((a.N + kTileCols - 1) / kTileCols, (P + kTileRows - 1) / kTileRows);
        hipLaunchKernelGGL(unpack_tile_kernel, grid, dim3(256), 0, stream, a);
    } else {
        dim3 grid((a.N + 255) / 256, P);
        hipLaunchKernelGGL(unpack_generic_kernel, grid, dim3(256), 0, stream, a);
    }
    return hipGetLastError();
}

}  // namespace ql
