/* main.m's copy of cpu_swiglu would clash with cpu_kernels.h's: rename it. */
#define cpu_swiglu main_m_cpu_swiglu
