// The IQ2_XXS codebook (the GGUF format's iq2xxs_grid; used by
// rsllm-gguf/src/dequant/iq2_xxs.rs:47-113 through iq2_xxs/tables.rs): 256
// entries of 8 magnitudes from {8, 25, 43}. Stored here as base-3 numbers
// (byte j of an entry = digit j; 8 -> 0, 25 -> 1, 43 -> 2) and expanded at
// compile time into the 8-byte entries the kernels index.
#pragma once

#include "common.h"

namespace rsllm_hip {

constexpr uint16_t kIq2Codes[256] = {
       0,    2,    4,    6,    8,   10,   12,   18,   20,   24,   26,   28,   30,   36,   42,   46,
      48,   54,   56,   62,   74,   82,   84,   90,   94,  108,  138,  150,  162,  164,  182,  218,
     244,  246,  252,  262,  264,  270,  272,  276,  288,  298,  300,  306,  318,  324,  326,  330,
     342,  356,  376,  378,  388,  412,  414,  432,  462,  480,  486,  490,  492,  498,  510,  514,
     516,  522,  524,  546,  570,  594,  650,  660,  730,  732,  738,  748,  756,  774,  786,  792,
     796,  810,  816,  828,  846,  854,  864,  912,  922,  972,  978,  990,  994, 1006, 1026, 1068,
    1100, 1134, 1148, 1216, 1218, 1224, 1242, 1270, 1296, 1300, 1368, 1414, 1458, 1460, 1466, 1488,
    1504, 1512, 1514, 1564, 1572, 1620, 1622, 1702, 1704, 1710, 1728, 1742, 1782, 1810, 1830, 1926,
    1950, 1962, 2010, 2136, 2188, 2190, 2196, 2202, 2206, 2208, 2214, 2220, 2228, 2232, 2242, 2244,
    2250, 2268, 2286, 2314, 2322, 2326, 2350, 2358, 2382, 2390, 2400, 2430, 2436, 2448, 2484, 2500,
    2522, 2532, 2592, 2674, 2676, 2682, 2700, 2704, 2754, 2796, 2800, 2810, 2866, 2898, 2916, 2922,
    2926, 2932, 2934, 2970, 2976, 3000, 3026, 3072, 3142, 3222, 3224, 3248, 3322, 3360, 3402, 3412,
    3418, 3450, 3510, 3570, 3648, 3654, 3672, 3696, 3726, 3766, 3822, 3852, 3888, 3892, 3978, 3980,
    4026, 4160, 4374, 4376, 4382, 4402, 4430, 4458, 4470, 4482, 4546, 4618, 4620, 4626, 4630, 4644,
    4662, 4698, 4730, 4764, 4786, 4806, 4824, 4862, 4944, 5032, 5106, 5112, 5124, 5130, 5176, 5198,
    5238, 5296, 5346, 5366, 5376, 5464, 5644, 5688, 5834, 5868, 5890, 5920, 5994, 6090, 6354, 6402,
};

constexpr uint64_t iq2_entry(uint32_t code) {
    uint64_t v = 0;
    for (int j = 0; j < 8; j++) {
        const uint32_t digit = code % 3;
        v |= (uint64_t)(digit == 0 ? 8 : digit == 1 ? 25 : 43) << (8 * j);
        code /= 3;
    }
    return v;
}

struct Iq2Grid {
    uint64_t v[256];
    constexpr Iq2Grid() : v() {
        for (int i = 0; i < 256; i++) v[i] = iq2_entry(kIq2Codes[i]);
    }
};

// Device copy (one per translation unit that includes this header).
static __constant__ Iq2Grid kIq2Grid = Iq2Grid();

// Sign byte of a 7-bit sign index: the index with bit 7 = its parity, so an
// even number of the 8 elements is negated (the format's ksigns table).
__device__ __forceinline__ uint32_t iq2_signs(uint32_t si) {
    return si | ((__builtin_popcount(si) & 1u) << 7);
}

}  // namespace rsllm_hip
