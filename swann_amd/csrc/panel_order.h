// Which row panel each workgroup of a symmetric-sweep band launch takes.
// Plain integer code, compiled for the device by the sweep and for the host
// by the CPU test that checks it is a permutation.
#pragma once

#if defined(__HIPCC__)
#define SWANN_HD __host__ __device__
#else
#define SWANN_HD
#endif

namespace swann {

// A band launch has one workgroup per row panel I in [0, g); panel I scores
// column tiles I + b0 .. I + b0 + B - 1 cut at the matrix edge, so the last B
// panels (the triangle) have B, B - 1, ... 1 tiles and the others B each.
// MI355X sends workgroup b to XCD b % 8 and each XCD runs its workgroups in
// order on its 32 CUs.  Equal contiguous runs of panels per XCD (xcd_remap)
// put the whole triangle on the last XCDs, which then idle while the others
// finish; panels spread round-robin balance the work but scatter neighbours,
// whose column tiles otherwise overlap one step apart and are re-read from
// the memory-side cache.  Here XCD x takes a contiguous run of the full-band
// panels [0, F) first, then every 8th triangle panel, F + 8 j + x: the same
// number of workgroups per XCD as the round-robin dispatch gives it, about
// the same work, and contiguous neighbours for all but the short tail.
SWANN_HD inline int sym_panel(int b, int g, int B) {
    const int x = b & 7, k = b >> 3;
    const int T = B < g ? B : g, F = g - T;
    // workgroups XCD y receives, and how many of them are triangle panels
    auto blocks = [&](int y) { return y < g ? (g - y + 7) >> 3 : 0; };
    auto tri = [&](int y) { return y < T ? (T - y + 7) >> 3 : 0; };
    const int full = blocks(x) - tri(x);
    if (k < full) {
        int start = 0;
        for (int y = 0; y < x; ++y) start += blocks(y) - tri(y);
        return start + k;
    }
    return F + (k - full) * 8 + x;
}

}  // namespace swann
