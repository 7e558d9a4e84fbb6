// SPDX-License-Identifier: MIT
// SHA-256 as specified in FIPS 180-4 section 6.2. The 64 round constants and
// the initial hash value are, by definition, the first 32 fractional bits of the
// cube roots of the first 64 primes and of the square roots of the first 8
// primes; they are derived here with exact integer roots instead of a table.
#include "ernie/sha256.h"

#include <cstring>

namespace ernie {
namespace {

using u128 = unsigned __int128;

// floor(x^(1/k)) for k = 2 or 3 and x < 2^108 (the inputs below stay far under that).
uint64_t integer_root(u128 x, int k)
{
    uint64_t lo = 0, hi = k == 2 ? (1ull << 54) : (1ull << 36);
    while (lo < hi) {
        const uint64_t mid = lo + (hi - lo + 1) / 2;
        u128 p = (u128)mid * mid;
        if (k == 3) p *= mid;
        if (p <= x) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

struct Constants {
    uint32_t k[64];
    uint32_t h0[8];
    Constants()
    {
        int primes[64];
        for (int n = 2, found = 0; found < 64; ++n) {
            bool prime = true;
            for (int d = 2; d * d <= n; ++d)
                if (n % d == 0) { prime = false; break; }
            if (prime) primes[found++] = n;
        }
        // frac(p^(1/3)) * 2^32 = low 32 bits of floor(cbrt(p * 2^96)); likewise sqrt with 2^64.
        for (int i = 0; i < 64; ++i) k[i] = (uint32_t)integer_root((u128)primes[i] << 96, 3);
        for (int i = 0; i < 8; ++i) h0[i] = (uint32_t)integer_root((u128)primes[i] << 64, 2);
    }
};

const Constants& constants()
{
    static const Constants c;
    return c;
}

inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

}  // namespace

Sha256::Sha256() { std::memcpy(h_, constants().h0, sizeof(h_)); }

void Sha256::block(const unsigned char* p)
{
    const uint32_t* K = constants().k;
    uint32_t w[64];
    for (int t = 0; t < 16; ++t)
        w[t] = (uint32_t)p[4 * t] << 24 | (uint32_t)p[4 * t + 1] << 16 | (uint32_t)p[4 * t + 2] << 8 | p[4 * t + 3];
    for (int t = 16; t < 64; ++t) {
        const uint32_t s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3);
        const uint32_t s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10);
        w[t] = w[t - 16] + s0 + w[t - 7] + s1;
    }
    uint32_t a = h_[0], b = h_[1], c = h_[2], d = h_[3], e = h_[4], f = h_[5], g = h_[6], h = h_[7];
    for (int t = 0; t < 64; ++t) {
        const uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
        const uint32_t ch = (e & f) ^ (~e & g);
        const uint32_t t1 = h + S1 + ch + K[t] + w[t];
        const uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
        const uint32_t maj = (a & b) ^ (a & c) ^ (b & c);
        const uint32_t t2 = S0 + maj;
        h = g; g = f; f = e; e = d + t1;
        d = c; c = b; b = a; a = t1 + t2;
    }
    h_[0] += a; h_[1] += b; h_[2] += c; h_[3] += d;
    h_[4] += e; h_[5] += f; h_[6] += g; h_[7] += h;
}

void Sha256::update(const void* data, size_t size)
{
    const unsigned char* p = static_cast<const unsigned char*>(data);
    total_ += size;
    if (used_) {
        const size_t take = size < 64 - used_ ? size : 64 - used_;
        std::memcpy(buf_ + used_, p, take);
        used_ += take;
        p += take;
        size -= take;
        if (used_ < 64) return;
        block(buf_);
        used_ = 0;
    }
    for (; size >= 64; p += 64, size -= 64) block(p);
    std::memcpy(buf_, p, size);
    used_ = size;
}

std::array<unsigned char, 32> Sha256::finish()
{
    const uint64_t bits = total_ * 8;
    const unsigned char one = 0x80, zero = 0;
    update(&one, 1);
    while (used_ != 56) update(&zero, 1);
    unsigned char len[8];
    for (int i = 0; i < 8; ++i) len[i] = (unsigned char)(bits >> (56 - 8 * i));
    update(len, 8);
    std::array<unsigned char, 32> out;
    for (int i = 0; i < 8; ++i)
        for (int j = 0; j < 4; ++j) out[4 * i + j] = (unsigned char)(h_[i] >> (24 - 8 * j));
    return out;
}

std::string Sha256::finish_hex()
{
    static const char hex[] = "0123456789abcdef";
    std::string s;
    for (unsigned char c : finish()) {
        s += hex[c >> 4];
        s += hex[c & 15];
    }
    return s;
}

std::string sha256_hex(const void* data, size_t size)
{
    Sha256 h;
    h.update(data, size);
    return h.finish_hex();
}

}  // namespace ernie
