// KV and state commitment hashing on the GPU (BLAKE3, gfx950 VALU).
//
// The commitment scheme of the reference (crates/qx-commit/src/state.rs) cuts a
// byte string into 256-byte chunks, hashes chunk i as
//   BLAKE3(domain || u64 4 || u32 i || u64 256 || chunk)        (hash_domain)
// and reduces the chunk digests pairwise with BLAKE3(left || right).  A KV leaf
// is BLAKE3("QX:KV:V1" || u64 2 || u16 layer || u64 4 || u32 token || u64 32 ||
// key_root || u64 32 || value_root).  Every hashed message fits one
// 1024-byte BLAKE3 chunk, so a digest is a short sequence of compressions of
// 64-byte blocks (chunk flags START on the first, END|ROOT on the last).
//
// In the head-major cache a token's K row (the reference's position-major
// [kv_head][d] bytes) is kv_heads pieces of head_dim elements, one per head.
// A lane hashes one 256-byte chunk of a row: it loads the chunk with sixteen
// 16-byte loads, assembles the message words in registers (the framing is
// compile-time except the chunk index) and runs five compressions.  The
// chunk digests of a row sit in a power-of-two group of adjacent lanes and
// are reduced with cross-lane shuffles; lane 0 of the group finishes the leaf.
// Every lane of a group runs every step (no divergence).  Per lane: 10
// compressions for its K and V chunks, one for the first tree level of both
// sides together, one per further level, two for the leaf: 14 for 4-chunk
// rows, the minimum for 16 leaves per wave.
#include "common.h"
#include "internal.h"

namespace qxh {

namespace {

constexpr uint32_t kFlagStart = 1, kFlagEnd = 2, kFlagRoot = 8;

struct Schedule {
    uint8_t w[7][16];
};
// message word order of each round: the BLAKE3 permutation applied r times
constexpr Schedule make_schedule() {
    Schedule s{};
    constexpr uint8_t perm[16] = {2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8};
    for (int i = 0; i < 16; ++i) s.w[0][i] = (uint8_t)i;
    for (int r = 1; r < 7; ++r)
        for (int i = 0; i < 16; ++i) s.w[r][i] = s.w[r - 1][perm[i]];
    return s;
}

__device__ __forceinline__ uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

__device__ __forceinline__ void mix(uint32_t& a, uint32_t& b, uint32_t& c, uint32_t& d, uint32_t x, uint32_t y) {
    a = a + b + x;
    d = rotr(d ^ a, 16);
    c = c + d;
    b = rotr(b ^ c, 12);
    a = a + b + y;
    d = rotr(d ^ a, 8);
    c = c + d;
    b = rotr(b ^ c, 7);
}

// One BLAKE3 compression (chunk counter 0); cv is updated in place.
__device__ __forceinline__ void compress(uint32_t (&cv)[8], const uint32_t (&m)[16], uint32_t block_len,
                                         uint32_t flags) {
    constexpr Schedule S = make_schedule();
    uint32_t v[16] = {cv[0],       cv[1],       cv[2],       cv[3],       cv[4], cv[5], cv[6],     cv[7],
                      0x6A09E667u, 0xBB67AE85u, 0x3C6EF372u, 0xA54FF53Au, 0u,    0u,    block_len, flags};
#pragma unroll
    for (int r = 0; r < 7; ++r) {
        mix(v[0], v[4], v[8], v[12], m[S.w[r][0]], m[S.w[r][1]]);
        mix(v[1], v[5], v[9], v[13], m[S.w[r][2]], m[S.w[r][3]]);
        mix(v[2], v[6], v[10], v[14], m[S.w[r][4]], m[S.w[r][5]]);
        mix(v[3], v[7], v[11], v[15], m[S.w[r][6]], m[S.w[r][7]]);
        mix(v[0], v[5], v[10], v[15], m[S.w[r][8]], m[S.w[r][9]]);
        mix(v[1], v[6], v[11], v[12], m[S.w[r][10]], m[S.w[r][11]]);
        mix(v[2], v[7], v[8], v[13], m[S.w[r][12]], m[S.w[r][13]]);
        mix(v[3], v[4], v[9], v[14], m[S.w[r][14]], m[S.w[r][15]]);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) cv[i] = v[i] ^ v[i + 8];
}

__device__ __forceinline__ void iv_init(uint32_t (&cv)[8]) {
    cv[0] = 0x6A09E667u; cv[1] = 0xBB67AE85u; cv[2] = 0x3C6EF372u; cv[3] = 0xA54FF53Au;
    cv[4] = 0x510E527Fu; cv[5] = 0x9B05688Cu; cv[6] = 0x1F83D9ABu; cv[7] = 0x5BE0CD19u;
}

// Framing of a 256-byte chunk leaf: domain || u64 4 || u32 index || u64 256,
// packed little-endian into words with the index bytes left zero.
struct Prefix {
    uint32_t w[12];
    int len;
};
template <int N>
constexpr Prefix make_prefix(const char (&domain)[N]) {
    Prefix p{};
    uint8_t b[48] = {};
    int n = 0;
    for (int i = 0; i < N - 1; ++i) b[n++] = (uint8_t)domain[i];
    b[n] = 4;          // u64 LE length of the index field
    n += 8;
    n += 4;            // u32 index (filled at run time)
    b[n + 1] = 1;      // u64 LE 256 = 00 01 00 .. 00
    n += 8;
    for (int i = 0; i < 12; ++i)
        p.w[i] = (uint32_t)b[4 * i] | ((uint32_t)b[4 * i + 1] << 8) | ((uint32_t)b[4 * i + 2] << 16) |
                 ((uint32_t)b[4 * i + 3] << 24);
    p.len = n;
    return p;
}

// Word w of the message stream prefix || chunk || zero padding (P = prefix
// bytes; everything but the chunk words is compile-time after unrolling).
// The chunk arrives as sixteen 16-byte groups g[0..15].
template <int P>
__device__ __forceinline__ uint32_t stream_word(int w, const uint32_t (&pw)[12], const u32x4 (&g)[16]) {
    auto cw = [&](int q) -> uint32_t { return q < 64 ? g[q >> 2][q & 3] : 0u; };
    const int b0 = 4 * w;
    if (b0 + 4 <= P) return pw[w];
    if (b0 < P) return pw[w] | (cw(0) << (8 * (P - b0)));
    const int s = b0 - P;
    if (s >= 256) return 0u;
    const int q = s >> 2, r = s & 3;
    if (r == 0) return cw(q);
    return (cw(q) >> (8 * r)) | (cw(q + 1) << (32 - 8 * r));
}

// last 16-byte chunk group that message block b reads (-1: none)
template <int P>
constexpr int last_group(int b) {
    const int hi = 64 * b + 63 - P;   // last chunk byte the block can touch
    return hi < 0 ? -1 : (hi >> 4) > 15 ? 15 : (hi >> 4);
}

// Leaf domains (crates/qx-commit/src/lib.rs:78-81)
struct StateChunkDomain {
    static constexpr int len = 17;
    static constexpr Prefix prefix() { return make_prefix("QX:STATE:CHUNK:V1"); }
};
struct KeyChunkDomain {
    static constexpr int len = 18;
    static constexpr Prefix prefix() { return make_prefix("QX:KV:KEY:CHUNK:V1"); }
};
struct ValueChunkDomain {
    static constexpr int len = 20;
    static constexpr Prefix prefix() { return make_prefix("QX:KV:VALUE:CHUNK:V1"); }
};

// BLAKE3 digest of one chunk leaf (chunk index idx).  load(i) returns bytes
// [16 i, 16 i + 16) of the chunk; each group is loaded once, one message
// block ahead of its first use, so only about two blocks' worth of chunk
// data is live at a time.
template <class Dom, class Load>
__device__ __forceinline__ void chunk_leaf(uint32_t idx, Load load, uint32_t (&out)[8]) {
    constexpr Prefix pre = Dom::prefix();
    constexpr int P = Dom::len + 20;
    static_assert(P == pre.len && P <= 48, "framing length");
    uint32_t pw[12];
#pragma unroll
    for (int i = 0; i < 12; ++i) pw[i] = pre.w[i];
    constexpr int ib = Dom::len + 8;   // first byte of the u32 index
    constexpr int sh = 8 * (ib % 4);
    pw[ib / 4] |= idx << sh;
    if constexpr (sh != 0) pw[ib / 4 + 1] |= idx >> (32 - sh);
    constexpr int total = P + 256;
    constexpr int blocks = (total + 63) / 64;
    u32x4 g[16];
#pragma unroll
    for (int i = 0; i <= last_group<P>(1); ++i) g[i] = load(i);
    iv_init(out);
#pragma unroll
    for (int b = 0; b < blocks; ++b) {
        if (b + 1 < blocks) {
#pragma unroll
            for (int i = last_group<P>(b + 1) + 1; i <= last_group<P>(b + 2); ++i) g[i] = load(i);
        }
        uint32_t m[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) m[i] = stream_word<P>(16 * b + i, pw, g);
        const uint32_t len = b + 1 < blocks ? 64u : (uint32_t)(total - 64 * (blocks - 1));
        const uint32_t flags = (b == 0 ? kFlagStart : 0u) | (b + 1 == blocks ? kFlagEnd | kFlagRoot : 0u);
        compress(out, m, len, flags);
    }
}

// The same digest with the chunk in two 128-byte pieces: the first (groups
// 0..7) is loaded into registers up front, the second (groups 8..15) was
// copied into LDS beforehand; staged(k) returns its group 8 + k.  Every
// group of a piece is requested in one burst, so each 128-byte line is
// fetched from HBM once; a line read piece by piece over several
// compressions may leave L2 in between and be fetched again.
template <class Dom, class Load, class Staged>
__device__ __forceinline__ void chunk_leaf_staged(uint32_t idx, Load load, Staged staged, uint32_t (&out)[8]) {
    constexpr Prefix pre = Dom::prefix();
    constexpr int P = Dom::len + 20;
    static_assert(P == pre.len && P <= 48, "framing length");
    static_assert(last_group<P>(0) < 8, "block 0 reads the first piece only");
    uint32_t pw[12];
#pragma unroll
    for (int i = 0; i < 12; ++i) pw[i] = pre.w[i];
    constexpr int ib = Dom::len + 8;
    constexpr int sh = 8 * (ib % 4);
    pw[ib / 4] |= idx << sh;
    if constexpr (sh != 0) pw[ib / 4 + 1] |= idx >> (32 - sh);
    constexpr int total = P + 256;
    constexpr int blocks = (total + 63) / 64;
    u32x4 g[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) g[i] = load(i);
    iv_init(out);
    bool landed = false;
#pragma unroll
    for (int b = 0; b < blocks; ++b) {
        // the staged groups of block b + 1, read one block ahead
        if (b + 1 < blocks) {
            const int lo = last_group<P>(b) + 1 > 8 ? last_group<P>(b) + 1 : 8;
            const int hi = last_group<P>(b + 1);
            if (hi >= lo && !landed) {
                // the copy into LDS was issued before the register loads
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                landed = true;
            }
#pragma unroll
            for (int i = lo; i <= hi; ++i) g[i] = staged(i - 8);
        }
        uint32_t m[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) m[i] = stream_word<P>(16 * b + i, pw, g);
        const uint32_t len = b + 1 < blocks ? 64u : (uint32_t)(total - 64 * (blocks - 1));
        const uint32_t flags = (b == 0 ? kFlagStart : 0u) | (b + 1 == blocks ? kFlagEnd | kFlagRoot : 0u);
        compress(out, m, len, flags);
    }
}

// parent = BLAKE3(left || right): one full block
__device__ __forceinline__ void parent_digest(const uint32_t (&l)[8], const uint32_t (&r)[8], uint32_t (&out)[8]) {
    uint32_t m[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        m[i] = l[i];
        m[8 + i] = r[i];
    }
    iv_init(out);
    compress(out, m, 64u, kFlagStart | kFlagEnd | kFlagRoot);
}

// Pairwise reduction of the digests held by a power-of-two group of `width`
// adjacent lanes (lane index within the group: gl).  Both lanes of a pair
// compute the parent, so after the loop every lane of the group holds the root.
__device__ __forceinline__ void group_tree(uint32_t (&d)[8], int gl, int width, int first = 1) {
    for (int lvl = first; lvl < width; lvl <<= 1) {
        uint32_t o[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = (uint32_t)__shfl_xor((int)d[i], lvl);
        uint32_t l[8], r[8];
        const bool left = (gl & lvl) == 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            l[i] = left ? d[i] : o[i];
            r[i] = left ? o[i] : d[i];
        }
        parent_digest(l, r, d);
    }
}

// K and V chunk digests of one row sit in a group of CH lanes (lane c holds
// chunk c of both).  The first tree level of both sides takes one compression
// per lane: lane c < CH/2 forms K node c from chunks 2c and 2c+1, lane
// c >= CH/2 forms V node c - CH/2.  The remaining levels reduce each half of
// the group; afterwards lanes [0, CH/2) hold the key root and lanes
// [CH/2, CH) the value root.
template <int CH>
__device__ __forceinline__ void kv_roots(const uint32_t (&kd)[8], const uint32_t (&vd)[8], int lane, int gl,
                                         uint32_t (&node)[8]) {
    constexpr int H = CH / 2;
    const bool vside = gl >= H;
    const int p = vside ? gl - H : gl;
    const int base = lane - gl;
    uint32_t l[8], r[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int lk = __shfl((int)kd[i], base + 2 * p), rk = __shfl((int)kd[i], base + 2 * p + 1);
        const int lv = __shfl((int)vd[i], base + 2 * p), rv = __shfl((int)vd[i], base + 2 * p + 1);
        l[i] = (uint32_t)(vside ? lv : lk);
        r[i] = (uint32_t)(vside ? rv : rk);
    }
    parent_digest(l, r, node);
    group_tree(node, p, H);
}

// KV leaf: BLAKE3("QX:KV:V1" || u64 2 || u16 layer || u64 4 || u32 token ||
// u64 32 || key_root || u64 32 || value_root), 110 bytes in two blocks.
__device__ __forceinline__ void kv_leaf(uint32_t layer, uint32_t token, const uint32_t (&kr)[8],
                                        const uint32_t (&vr)[8], uint32_t (&out)[8]) {
    uint32_t w[32] = {};
    w[0] = 0x4B3A5851u;  // "QX:K"
    w[1] = 0x31563A56u;  // "V:V1"
    w[2] = 2u;                                   // bytes 8..15: u64 2
    w[4] = (layer & 0xffffu) | (4u << 16);       // 16..17 layer, 18..25: u64 4
    w[6] = (token & 0xffffu) << 16;              // 26..29 token
    w[7] = (token >> 16) | (32u << 16);          // 30..37: u64 32
    w[9] = kr[0] << 16;                          // 38..69 key root
#pragma unroll
    for (int j = 1; j < 8; ++j) w[9 + j] = (kr[j - 1] >> 16) | (kr[j] << 16);
    w[17] = (kr[7] >> 16) | (32u << 16);         // 70..77: u64 32
    w[19] = vr[0] << 16;                         // 78..109 value root
#pragma unroll
    for (int j = 1; j < 8; ++j) w[19 + j] = (vr[j - 1] >> 16) | (vr[j] << 16);
    w[27] = vr[7] >> 16;
    uint32_t m0[16], m1[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        m0[i] = w[i];
        m1[i] = w[16 + i];
    }
    iv_init(out);
    compress(out, m0, 64u, kFlagStart);
    compress(out, m1, 46u, kFlagEnd | kFlagRoot);
}

// Byte address of row byte o of a token row [kv_head][head_bytes] in the
// head-major layer base (o is a multiple of 16).
__device__ __forceinline__ const char* row_byte(const char* base, uint64_t head_stride_bytes, uint32_t head_shift,
                                                uint64_t row_off, uint32_t o) {
    const uint32_t head = o >> head_shift, within = o & ((1u << head_shift) - 1u);
    return base + head * head_stride_bytes + row_off + within;
}

__device__ __forceinline__ void store_digest(uint8_t* dst, const uint32_t (&d)[8]) {
    u32x4* p = reinterpret_cast<u32x4*>(dst);
    p[0] = u32x4{d[0], d[1], d[2], d[3]};
    p[1] = u32x4{d[4], d[5], d[6], d[7]};
}

}  // namespace

// ---------------------------------------------------------------------------
// bulk KV leaves: out[s][i] = kv_leaf_hash_v1(layer, token_begin + i, K row, V row)
// ---------------------------------------------------------------------------
struct KvLeafArgs {
    const char* keys;            // layer base of the first sequence
    const char* values;
    uint64_t head_stride_bytes_k;
    uint64_t head_stride_bytes_v;
    uint64_t seq_stride_bytes_k;
    uint64_t seq_stride_bytes_v;
    uint32_t head_shift_k;       // log2(head_dim * element bytes)
    uint32_t head_shift_v;
    uint32_t token_begin;
    uint32_t count;
    uint32_t sequences;
    uint32_t layer;
    uint8_t* out;
};

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void global_void;

// Copy bytes [128, 256) of a lane's chunk into LDS: eight 16-byte
// direct-to-LDS loads, group 8 + k of lane l landing at stage[k][l].
template <class Addr>
__device__ __forceinline__ void stage_second_piece(Addr addr, u32x4 (*stage)[64]) {
#pragma unroll
    for (int k = 0; k < 8; ++k)
        __builtin_amdgcn_global_load_lds((global_void*)addr(8 + k), (lds_void*)&stage[k][0], 16, 0, 0);
}

// CH = chunks per row (4 or 8): 64 / CH leaves per wave, 4 waves per block.
// Each wave stages the second half of its lanes' chunks in 8 KB of LDS
// (32 KB per block, three blocks per CU).
template <int CH>
__global__ __launch_bounds__(256, 3) void kv_leaf_hash_kernel(KvLeafArgs a) {
    __shared__ u32x4 stage_all[4][8][64];
    constexpr int LPW = 64 / CH;
    const int lane = threadIdx.x & 63;
    const int gl = lane % CH;
    u32x4 (*stage)[64] = stage_all[__builtin_amdgcn_readfirstlane(threadIdx.x >> 6)];
    const uint64_t total = (uint64_t)a.sequences * a.count;
    const uint64_t leaf = ((uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * LPW + lane / CH;
    const bool live = leaf < total;
    const uint64_t lf = live ? leaf : total - 1;  // spare lanes repeat the last leaf and store nothing
    const uint32_t s = (uint32_t)(lf / a.count), i = (uint32_t)(lf % a.count);
    const uint32_t tok = a.token_begin + i;
    const uint64_t row_off = (uint64_t)tok << a.head_shift_k;
    const char* kb = a.keys + s * a.seq_stride_bytes_k;
    const char* vb = a.values + s * a.seq_stride_bytes_v;
    uint32_t kd[8], vd[8], node[8], d[8];
    auto kaddr = [&](int i) { return row_byte(kb, a.head_stride_bytes_k, a.head_shift_k, row_off, 256u * gl + 16u * i); };
    auto vaddr = [&](int i) { return row_byte(vb, a.head_stride_bytes_v, a.head_shift_v, row_off, 256u * gl + 16u * i); };
    auto staged = [&](int k) { return stage[k][lane]; };
    stage_second_piece(kaddr, stage);
    chunk_leaf_staged<KeyChunkDomain>((uint32_t)gl, [&](int i) { return *reinterpret_cast<const u32x4*>(kaddr(i)); },
                                      staged, kd);
    // every LDS read of the key piece has returned before the value piece lands there
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    stage_second_piece(vaddr, stage);
    chunk_leaf_staged<ValueChunkDomain>((uint32_t)gl, [&](int i) { return *reinterpret_cast<const u32x4*>(vaddr(i)); },
                                        staged, vd);
    kv_roots<CH>(kd, vd, lane, gl, node);
    // lane 0 of the group: key root; lane CH/2: value root
    uint32_t vr[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) vr[i] = (uint32_t)__shfl((int)node[i], lane - gl + CH / 2);
    kv_leaf(a.layer, tok, node, vr, d);
    if (live && gl == 0) store_digest(a.out + leaf * 32, d);
}

// K and V rows of different sizes (KvPrecision Fp32KFp16V / Fp16KFp32V,
// crates/qx-format/src/lib.rs:136-141): a group of CH = max(CHK, CHV) lanes
// per leaf; lane c hashes K chunk c (c < CHK) and V chunk c (c < CHV), spare
// lanes repeat chunk 0, and the two trees reduce separately.
template <int CHK, int CHV>
__global__ __launch_bounds__(256, 3) void kv_leaf_hash_mixed_kernel(KvLeafArgs a) {
    constexpr int CH = CHK > CHV ? CHK : CHV;
    constexpr int LPW = 64 / CH;
    const int lane = threadIdx.x & 63;
    const int gl = lane % CH;
    const uint64_t total = (uint64_t)a.sequences * a.count;
    const uint64_t leaf = ((uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * LPW + lane / CH;
    const bool live = leaf < total;
    const uint64_t lf = live ? leaf : total - 1;
    const uint32_t s = (uint32_t)(lf / a.count), i = (uint32_t)(lf % a.count);
    const uint32_t tok = a.token_begin + i;
    const char* kb = a.keys + s * a.seq_stride_bytes_k;
    const char* vb = a.values + s * a.seq_stride_bytes_v;
    const uint64_t koff = (uint64_t)tok << a.head_shift_k, voff = (uint64_t)tok << a.head_shift_v;
    const uint32_t ck = gl < CHK ? (uint32_t)gl : 0u, cv = gl < CHV ? (uint32_t)gl : 0u;
    uint32_t kd[8], vd[8], d[8];
    chunk_leaf<KeyChunkDomain>(ck, [&](int i) {
        return *reinterpret_cast<const u32x4*>(row_byte(kb, a.head_stride_bytes_k, a.head_shift_k, koff, 256u * ck + 16u * i));
    }, kd);
    chunk_leaf<ValueChunkDomain>(cv, [&](int i) {
        return *reinterpret_cast<const u32x4*>(row_byte(vb, a.head_stride_bytes_v, a.head_shift_v, voff, 256u * cv + 16u * i));
    }, vd);
    group_tree(kd, gl, CHK);
    group_tree(vd, gl, CHV);
    kv_leaf(a.layer, tok, kd, vd, d);
    if (live && gl == 0) store_digest(a.out + leaf * 32, d);
}

// ---------------------------------------------------------------------------
// per-token verification digests (kernels/verification_hash.metal:349-522):
// block p = 0..layers; wave 0 hashes the residual snapshot p (checkpoint
// layers and genesis), waves 1 and 2 the K and V rows of layer p-1.
// ---------------------------------------------------------------------------
struct VerifyArgs {
    const char* residuals;       // [(layers + 1)][residual_stride]
    const char* keys;            // layer 0, this sequence
    const char* values;
    uint64_t layer_stride_bytes_k;
    uint64_t layer_stride_bytes_v;
    uint64_t head_stride_bytes_k;
    uint64_t head_stride_bytes_v;
    uint32_t head_shift_k;
    uint32_t head_shift_v;
    uint32_t k_chunks;           // chunks per K row
    uint32_t v_chunks;           // chunks per V row
    uint32_t residual_stride;
    uint32_t state_chunks;
    uint32_t token;
    uint32_t layers;
    uint32_t interval;
    uint8_t* out;                // [(layers + 1)][64]
};

__global__ __launch_bounds__(192) void verification_hash_kernel(VerifyArgs a) {
    __shared__ uint32_t roots[3][8];
    const uint32_t p = blockIdx.x;
    const bool genesis = p == 0;
    const uint32_t layer = genesis ? 0u : p - 1u;
    const bool checkpoint = genesis || (layer + 1u) % a.interval == 0u || layer + 1u == a.layers;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    uint32_t d[8];
    if (wave == 0) {
        if (checkpoint) {
            const uint32_t gl = (uint32_t)lane < a.state_chunks ? (uint32_t)lane : 0u;
            const char* src = a.residuals + (uint64_t)p * a.residual_stride + 256u * gl;
            chunk_leaf<StateChunkDomain>(gl, [&](int i) { return *reinterpret_cast<const u32x4*>(src + 16 * i); }, d);
            group_tree(d, lane, (int)a.state_chunks);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) d[i] = 0u;
        }
    } else if (!genesis) {
        const bool key = wave == 1;
        const uint32_t chunks = key ? a.k_chunks : a.v_chunks;
        const uint32_t gl = (uint32_t)lane < chunks ? (uint32_t)lane : 0u;
        const uint32_t shift = key ? a.head_shift_k : a.head_shift_v;
        const char* base = key ? a.keys + layer * a.layer_stride_bytes_k : a.values + layer * a.layer_stride_bytes_v;
        const uint64_t hs = key ? a.head_stride_bytes_k : a.head_stride_bytes_v;
        const uint64_t row_off = (uint64_t)a.token << shift;
        auto load = [&](int i) {
            return *reinterpret_cast<const u32x4*>(row_byte(base, hs, shift, row_off, 256u * gl + 16u * i));
        };
        if (key) chunk_leaf<KeyChunkDomain>(gl, load, d);
        else chunk_leaf<ValueChunkDomain>(gl, load, d);
        group_tree(d, lane, (int)chunks);
    }
    if (lane == 0 && (wave == 0 || !genesis)) {
#pragma unroll
        for (int i = 0; i < 8; ++i) roots[wave][i] = d[i];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint8_t* o = a.out + (uint64_t)p * 64;
        uint32_t sr[8], kr[8], vr[8], leaf[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            sr[i] = roots[0][i];
            kr[i] = roots[1][i];
            vr[i] = roots[2][i];
        }
        store_digest(o, sr);
        if (genesis) {
#pragma unroll
            for (int i = 0; i < 8; ++i) leaf[i] = 0u;
        } else {
            kv_leaf(layer, a.token, kr, vr, leaf);
        }
        store_digest(o + 32, leaf);
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static uint32_t log2u(uint64_t v) {
    uint32_t s = 0;
    while ((1ull << s) < v) ++s;
    return s;
}

hipError_t launch_kv_leaf_hashes(const ShapeDims& s, const KvLayer& kv, uint32_t layer, uint32_t sequences,
                                 uint32_t token_begin, uint32_t count, void* out, hipStream_t st) {
    const uint32_t ebk = kv.key_dtype == F32 ? 4u : 2u, ebv = kv.value_dtype == F32 ? 4u : 2u;
    KvLeafArgs a{};
    a.keys = reinterpret_cast<const char*>(kv.keys);
    a.values = reinterpret_cast<const char*>(kv.values);
    a.head_stride_bytes_k = kv.head_stride * ebk;
    a.head_stride_bytes_v = kv.head_stride * ebv;
    a.seq_stride_bytes_k = kv.sequence_stride * ebk;
    a.seq_stride_bytes_v = kv.sequence_stride * ebv;
    a.head_shift_k = log2u((uint64_t)s.head_dim * ebk);
    a.head_shift_v = log2u((uint64_t)s.head_dim * ebv);
    a.token_begin = token_begin;
    a.count = count;
    a.sequences = sequences;
    a.layer = layer;
    a.out = reinterpret_cast<uint8_t*>(out);
    const uint64_t leaves = (uint64_t)sequences * count;
    const uint32_t chk = (uint32_t)((uint64_t)s.head_dim * ebk * s.kv_heads / 256);
    const uint32_t chv = (uint32_t)((uint64_t)s.head_dim * ebv * s.kv_heads / 256);
    const uint32_t ch = chk > chv ? chk : chv;
    const uint64_t per_block = 4ull * (64 / ch);
    const dim3 grid((uint32_t)((leaves + per_block - 1) / per_block));
    if (chk == 4 && chv == 4) hipLaunchKernelGGL(kv_leaf_hash_kernel<4>, grid, dim3(256), 0, st, a);
    else if (chk == 8 && chv == 8) hipLaunchKernelGGL(kv_leaf_hash_kernel<8>, grid, dim3(256), 0, st, a);
    else if (chk == 8 && chv == 4) hipLaunchKernelGGL((kv_leaf_hash_mixed_kernel<8, 4>), grid, dim3(256), 0, st, a);
    else if (chk == 4 && chv == 8) hipLaunchKernelGGL((kv_leaf_hash_mixed_kernel<4, 8>), grid, dim3(256), 0, st, a);
    else return hipErrorNotSupported;
    return hipGetLastError();
}

hipError_t launch_verification_hashes(const ShapeDims& s, const KvLayer& kv0, uint64_t layer_stride_elems,
                                      const void* residuals, uint32_t residual_stride, uint32_t token, uint32_t layers,
                                      uint32_t interval, void* out, hipStream_t st) {
    const uint32_t ebk = kv0.key_dtype == F32 ? 4u : 2u, ebv = kv0.value_dtype == F32 ? 4u : 2u;
    VerifyArgs a{};
    a.residuals = reinterpret_cast<const char*>(residuals);
    a.keys = reinterpret_cast<const char*>(kv0.keys);
    a.values = reinterpret_cast<const char*>(kv0.values);
    a.layer_stride_bytes_k = layer_stride_elems * ebk;
    a.layer_stride_bytes_v = layer_stride_elems * ebv;
    a.head_stride_bytes_k = kv0.head_stride * ebk;
    a.head_stride_bytes_v = kv0.head_stride * ebv;
    a.head_shift_k = log2u((uint64_t)s.head_dim * ebk);
    a.head_shift_v = log2u((uint64_t)s.head_dim * ebv);
    a.k_chunks = (uint32_t)((uint64_t)s.head_dim * ebk * s.kv_heads / 256);
    a.v_chunks = (uint32_t)((uint64_t)s.head_dim * ebv * s.kv_heads / 256);
    a.residual_stride = residual_stride;
    a.state_chunks = residual_stride / 256;
    a.token = token;
    a.layers = layers;
    a.interval = interval;
    a.out = reinterpret_cast<uint8_t*>(out);
    hipLaunchKernelGGL(verification_hash_kernel, dim3(layers + 1), dim3(192), 0, st, a);
    return hipGetLastError();
}

}  // namespace qxh
