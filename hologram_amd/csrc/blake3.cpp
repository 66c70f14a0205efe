// blake3.cpp — BLAKE3 (the published algorithm: 1024-byte chunks of 64-byte
// blocks, a binary Merkle tree of chaining values, 7-round compression with
// the BLAKE2s message schedule) in portable C++. Used for the `.holo` footer
// fingerprint (crates/hologram-archive/src/loader.rs:161-179, writer.rs
// `assemble`) and the Weights-section fingerprints (weight.rs
// `WeightFingerprint::of`). Default hash mode, 32-byte output only.
//
// Whole chunks are hashed on worker threads when the input is large (the
// chunk chaining values are independent); the tree is then folded in the
// same order as the sequential algorithm, so the digest does not depend on
// the thread count.
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <thread>
#include <vector>

namespace holo {
namespace {

constexpr uint32_t kIV[8] = {0x6A09E667u, 0xBB67AE85u, 0x3C6EF372u, 0xA54FF53Au,
                             0x510E527Fu, 0x9B05688Cu, 0x1F83D9ABu, 0x5BE0CD19u};
constexpr uint8_t kPerm[16] = {2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8};
constexpr uint32_t CHUNK_START = 1, CHUNK_END = 2, PARENT = 4, ROOT = 8;
constexpr size_t kChunk = 1024, kBlock = 64;

inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

inline void g(uint32_t *s, int a, int b, int c, int d, uint32_t x, uint32_t y) {
    s[a] = s[a] + s[b] + x;
    s[d] = rotr(s[d] ^ s[a], 16);
    s[c] = s[c] + s[d];
    s[b] = rotr(s[b] ^ s[c], 12);
    s[a] = s[a] + s[b] + y;
    s[d] = rotr(s[d] ^ s[a], 8);
    s[c] = s[c] + s[d];
    s[b] = rotr(s[b] ^ s[c], 7);
}

// The compression function; writes the first 8 words of the output state.
void compress(const uint32_t cv[8], const uint32_t block[16], uint64_t counter, uint32_t len,
              uint32_t flags, uint32_t out[8]) {
    uint32_t s[16] = {cv[0], cv[1], cv[2], cv[3], cv[4], cv[5], cv[6], cv[7],
                      kIV[0], kIV[1], kIV[2], kIV[3], uint32_t(counter), uint32_t(counter >> 32),
                      len, flags};
    uint32_t m[16];
    memcpy(m, block, sizeof(m));
    for (int r = 0; r < 7; ++r) {
        g(s, 0, 4, 8, 12, m[0], m[1]);
        g(s, 1, 5, 9, 13, m[2], m[3]);
        g(s, 2, 6, 10, 14, m[4], m[5]);
        g(s, 3, 7, 11, 15, m[6], m[7]);
        g(s, 0, 5, 10, 15, m[8], m[9]);
        g(s, 1, 6, 11, 12, m[10], m[11]);
        g(s, 2, 7, 8, 13, m[12], m[13]);
        g(s, 3, 4, 9, 14, m[14], m[15]);
        if (r < 6) {
            uint32_t t[16];
            for (int i = 0; i < 16; ++i) t[i] = m[kPerm[i]];
            memcpy(m, t, sizeof(m));
        }
    }
    for (int i = 0; i < 8; ++i) out[i] = s[i] ^ s[i + 8];
}

void load_block(const uint8_t *p, size_t n, uint32_t w[16]) {
    uint8_t buf[kBlock] = {};
    memcpy(buf, p, n);
    for (int i = 0; i < 16; ++i)
        w[i] = uint32_t(buf[4 * i]) | uint32_t(buf[4 * i + 1]) << 8 |
               uint32_t(buf[4 * i + 2]) << 16 | uint32_t(buf[4 * i + 3]) << 24;
}

// Chaining value of chunk `index` (n <= 1024 bytes). `root`: the chunk is the
// whole input, so its last block carries ROOT.
void chunk_cv(const uint8_t *p, size_t n, uint64_t index, bool root, uint32_t out[8]) {
    uint32_t cv[8];
    memcpy(cv, kIV, sizeof(cv));
    const size_t nblocks = n == 0 ? 1 : (n + kBlock - 1) / kBlock;
    for (size_t b = 0; b < nblocks; ++b) {
        const size_t off = b * kBlock;
        const size_t len = std::min(kBlock, n - std::min(n, off));
        uint32_t w[16];
        load_block(p + off, len, w);
        uint32_t flags = 0;
        if (b == 0) flags |= CHUNK_START;
        if (b + 1 == nblocks) flags |= CHUNK_END | (root ? ROOT : 0);
        compress(cv, w, index, uint32_t(len), flags, cv);
    }
    memcpy(out, cv, sizeof(cv));
}

void parent_cv(const uint32_t l[8], const uint32_t r[8], bool root, uint32_t out[8]) {
    uint32_t w[16];
    memcpy(w, l, 32);
    memcpy(w + 8, r, 32);
    compress(kIV, w, 0, kBlock, PARENT | (root ? ROOT : 0), out);
}

}  // namespace

void blake3_hash(const void *data, size_t len, uint8_t out[32]) {
    const uint8_t *p = static_cast<const uint8_t *>(data);
    uint32_t root[8];
    if (len <= kChunk) {
        chunk_cv(p, len, 0, true, root);
    } else {
        const size_t nchunks = (len + kChunk - 1) / kChunk;
        std::vector<uint32_t> cvs(nchunks * 8);
        auto work = [&](size_t c0, size_t c1) {
            for (size_t c = c0; c < c1; ++c) {
                const size_t off = c * kChunk;
                chunk_cv(p + off, std::min(kChunk, len - off), c, false, &cvs[8 * c]);
            }
        };
        unsigned nt = nchunks >= 4096 ? std::min(16u, std::max(1u, std::thread::hardware_concurrency())) : 1u;
        if (nt <= 1) {
            work(0, nchunks);
        } else {
            std::vector<std::thread> ts;
            const size_t per = (nchunks + nt - 1) / nt;
            for (unsigned t = 0; t < nt; ++t) {
                const size_t a = std::min(nchunks, t * per), b = std::min(nchunks, a + per);
                if (a < b) ts.emplace_back(work, a, b);
            }
            for (auto &t : ts) t.join();
        }
        // Fold the chunk chaining values as the incremental hasher does: a
        // stack of subtree CVs, merged whenever the chunk count has a trailing
        // zero bit; the root is the final merge of the stack.
        std::vector<uint32_t> stack;
        for (size_t c = 0; c + 1 < nchunks; ++c) {
            uint32_t cv[8];
            memcpy(cv, &cvs[8 * c], 32);
            uint64_t total = c + 1;
            while ((total & 1) == 0) {
                uint32_t merged[8];
                parent_cv(&stack[stack.size() - 8], cv, false, merged);
                stack.resize(stack.size() - 8);
                memcpy(cv, merged, 32);
                total >>= 1;
            }
            stack.insert(stack.end(), cv, cv + 8);
        }
        uint32_t cv[8];
        memcpy(cv, &cvs[8 * (nchunks - 1)], 32);
        while (!stack.empty()) {
            uint32_t merged[8];
            parent_cv(&stack[stack.size() - 8], cv, stack.size() == 8, merged);
            stack.resize(stack.size() - 8);
            memcpy(cv, merged, 32);
        }
        memcpy(root, cv, 32);
    }
    for (int i = 0; i < 8; ++i) {
        out[4 * i] = uint8_t(root[i]);
        out[4 * i + 1] = uint8_t(root[i] >> 8);
        out[4 * i + 2] = uint8_t(root[i] >> 16);
        out[4 * i + 3] = uint8_t(root[i] >> 24);
    }
}

}  // namespace holo
