#ifndef CTORCH_AMD_EXPORT_H
#define CTORCH_AMD_EXPORT_H
/* Symbol visibility for the shared library (the reference's generated export header plays this role). */
#if defined(_WIN32)
#define DL_API __declspec(dllexport)
#else
#define DL_API __attribute__((visibility("default")))
#endif
#endif
