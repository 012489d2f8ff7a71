// Single translation unit of the shared library (the kernels share one
// device error word without relocatable device code).
#include "ffn_decode.hip"
#include "route.hip"
#include "grouped.hip"
#include "stack_decode.hip"
#include "capi.hip"
#include "engine.hip"
#include "policy.cpp"
