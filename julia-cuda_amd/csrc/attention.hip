// FlashAttention-2-style attention on MFMA (gfx950), global or sliding-window, heads of 64:
// o = softmax(q . k^T / 8) . v, keys |i - j| <= window (all keys when window is 0). The
// reference's kernel is kernels/src/main.rs:301-542 with attn.rs's building blocks.
//
// A block takes 64 queries of one head: four waves of 16. Keys go 64 at a time: K into an LDS
// tile [key][d], V transposed into [d][key]. Each wave computes S^T = K . Q^T (the MFMA's output
// gives lane l query l % 16 and 16 of the block's 64 keys), so the running max and sum need only
// in-lane work plus two cross-lane steps, and the lane's P values are exactly the B operand of
// O^T = V^T . P^T, whose output again gives lane l query l % 16 (16 of its 64 dimensions): the
// rescale by the new max is per lane. Softmax in the exp2 domain (scale log2(e) / 8); P rounded
// to f16 for P . V; f32 sums. Rows with no key in range get zeros.
//
// With `chunks` > 1 the key blocks of each (query block, head) tile are split into ranges, one
// block each; every range writes its unnormalised output, max and sum to the scratch and the
// last one of the tile to arrive merges them in range order (kernels/src/attn.rs:92-204).
#include <stdexcept>
#include <string>

#include "attn_tile.h"

namespace jh {

__global__ __launch_bounds__(256) void attention_kernel(AttnParams p) {
    __shared__ __attribute__((aligned(16))) f16 lds[ATT_LDS_F16];
    __shared__ uint32_t s_last;
    attention_tile(p, blockIdx.x, blockIdx.y, blockIdx.z, lds, &s_last);
}

size_t attention_ws_floats(int n, int d, int chunks) {
    if (chunks <= 1) return 0;
    return (size_t)((n + 63) / 64) * (d / 64) * chunks * ATT_PART * 256;
}

size_t attention_counters(int n, int d) { return (size_t)((n + 63) / 64) * (d / 64); }

// Key ranges per tile: split while the tiles don't fill the GPU, at least two key blocks a range
// (the reference's default_plan rule, src/forward.rs:186-187, refit for a 256-CU GPU).
int attention_chunks(int n, int d, int window, int cus) {
    if (window > 0) return 1;  // a window tile reaches 3 key blocks: splitting doesn't pay
    const int blocks = (n + 63) / 64, tiles = blocks * (d / 64);
    int c = (cus > 0 ? cus : 256) / (tiles > 0 ? tiles : 1);
    c = std::min(c, (blocks + 1) / 2);
    return std::max(1, std::min(c, 8));
}

void attention_launch(const jh_half* qkv, jh_half* o, int n, int d, int window, int chunks,
                      const Scratch& s, hipStream_t st) {
    auto fail = [](const std::string& m) { throw std::runtime_error("attention: " + m); };
    if (n <= 0) fail("no rows");
    if (d <= 0 || d % 64) fail("d = " + std::to_string(d) + " is not a multiple of 64");
    if (window < 0) fail("negative window");
    if (!qkv || !o || ((uintptr_t)qkv % 16) || ((uintptr_t)o % 16)) fail("qkv and o must be 16-byte aligned");
    if (chunks < 1 || chunks > 16) fail(std::to_string(chunks) + " key ranges");
    if (chunks > 1 && (attention_ws_floats(n, d, chunks) > s.ws_floats ||
                       attention_counters(n, d) > s.n_counters || !s.ws || !s.counters))
        fail("the key-range scratch is too small for " + std::to_string(n) + " tokens");
    AttnParams p{qkv, o, n, d, window, chunks, s.ws, s.counters};
    hipLaunchKernelGGL(attention_kernel, dim3((n + 63) / 64, d / 64, chunks), dim3(256), 0, st, p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) throw std::runtime_error(std::string("attention: ") + hipGetErrorString(e));
}

}  // namespace jh
