using System.Runtime.InteropServices;

namespace Llmdot.Hip.Native;

/// <summary>
/// P/Invoke declarations of libllmdot_hip.so, one per function of
/// include/llmdot_hip.h (same names, argument order and meaning).  Every
/// function returns an LLMDOT_* status code; <see cref="Check"/> turns a
/// failure into the exception the reference throws for the same condition.
/// </summary>
internal static unsafe partial class HipNative
{
    private const string Lib = "llmdot_hip";

    public const int Ok = 0;
    public const int EInvalid = -1;      // ArgumentException
    public const int EUnsupported = -2;  // NotSupportedException
    public const int ENotFound = -3;     // KeyNotFoundException
    public const int ERange = -4;        // ArgumentOutOfRangeException
    public const int EDevice = -5;       // HIP runtime error / no device
    public const int ENoMem = -6;        // device or host allocation failed

    [StructLayout(LayoutKind.Sequential)]
    public struct DeviceInfo
    {
        public fixed byte Name[64];
        public fixed byte Arch[32];
        public int ComputeUnits;
        public int ClockMhz;
        public ulong HbmBytes;
    }

    /// <summary>llmdot_hip_sampling: SamplingOptions without the seed (the caller draws).</summary>
    [StructLayout(LayoutKind.Sequential)]
    public struct Sampling
    {
        public float Temperature;
        public int TopK;
        public float TopP;
        public float RepeatPenalty;
        public int RepeatWindow;
    }

    /// <summary>llmdot_hip_model_desc: the TransformerConfig fields the decode step reads.</summary>
    [StructLayout(LayoutKind.Sequential)]
    public struct ModelDesc
    {
        public int Hidden;
        public int Layers;
        public int Heads;
        public int KvHeads;
        public int HeadDim;
        public int Ffn;
        public int Vocab;
        public int Context;
        public int RopeDim;
        public float Eps;
        public float RopeBase;
        public float RopeLinearFactor;
        public int KvFp16;
        public int Bos;
        public int SlidingWindow; // attend to the last N positions (IE:385-387); 0 = all
        public byte* KeyPrefix;   // NUL-terminated UTF-8, may be null
    }

    [StructLayout(LayoutKind.Sequential)]
    public struct StepTiming
    {
        public float TotalMs;
        public float GemvMs;
        public int GemvLaunches;
        public double GemvBytes;
    }

    // ---- context -----------------------------------------------------------
    [DllImport(Lib)] public static extern nint llmdot_hip_last_error();
    [DllImport(Lib)] public static extern int llmdot_hip_device_count(int* count);
    [DllImport(Lib)] public static extern int llmdot_hip_create(int device, nint* ctx);
    [DllImport(Lib)] public static extern int llmdot_hip_destroy(nint ctx);
    [DllImport(Lib)] public static extern int llmdot_hip_get_device_info(nint ctx, DeviceInfo* info);

    // ---- persistent weights --------------------------------------------------
    [DllImport(Lib)] public static extern int llmdot_hip_upload_weight(nint ctx, byte* key, uint ggmlType, void* bytes, nuint nbytes, long rows, long cols);
    [DllImport(Lib)] public static extern int llmdot_hip_release_weight(nint ctx, byte* key);
    [DllImport(Lib)] public static extern int llmdot_hip_has_weight(nint ctx, byte* key, int* present);

    // ---- op level (IComputeBackend) -------------------------------------------
    [DllImport(Lib)] public static extern int llmdot_hip_matmul(nint ctx, float* a, void* b, float* result, long resultLen, uint bType, int aCols, int bCols, byte* weightKey);
    [DllImport(Lib)] public static extern int llmdot_hip_matmul_f32(nint ctx, float* a, float* b, float* result, long resultLen, int aCols, int bCols, byte* weightKey);
    [DllImport(Lib)] public static extern int llmdot_hip_rms_norm(nint ctx, float* input, float* weights, float* output, int n, float epsilon);
    [DllImport(Lib)] public static extern int llmdot_hip_apply_rope(nint ctx, float* query, float* key, int headDim, int position, float* freqTable, int halfDim, int sameSpan);
    [DllImport(Lib)] public static extern int llmdot_hip_apply_rope_base(nint ctx, float* query, float* key, int headDim, int position, float freqBase, int rotaryDim, int sameSpan);
    [DllImport(Lib)] public static extern int llmdot_hip_softmax(nint ctx, float* input, int n, int hasSoftcap, float softcap);
    [DllImport(Lib)] public static extern int llmdot_hip_silu(nint ctx, float* input, float* result, int n);
    [DllImport(Lib)] public static extern int llmdot_hip_layer_norm(nint ctx, float* input, float* weights, float* biasOrNull, float* output, int n, float epsilon);
    [DllImport(Lib)] public static extern int llmdot_hip_gelu(nint ctx, float* input, float* result, int n);
    [DllImport(Lib)] public static extern int llmdot_hip_softcap(nint ctx, float* input, int n, float cap);
    [DllImport(Lib)] public static extern int llmdot_hip_conv1d(nint ctx, float* input, float* weights, float* output, int kernelSize, int inputDim);
    [DllImport(Lib)] public static extern int llmdot_hip_add(nint ctx, float* a, float* b, float* result, int n);
    [DllImport(Lib)] public static extern int llmdot_hip_scale(nint ctx, float* input, float scale, float* result, int n);
    [DllImport(Lib)] public static extern int llmdot_hip_mul(nint ctx, float* a, float* b, float* result, int n);
    [DllImport(Lib)] public static extern int llmdot_hip_dequantize(nint ctx, void* src, float* dst, uint ggmlType, int numRows, int rowElements);
    [DllImport(Lib)] public static extern int llmdot_hip_argmax(nint ctx, float* input, int n, int* index);
    [DllImport(Lib)] public static extern int llmdot_hip_sample(nint ctx, float* logits, int n, Sampling* opt, int* recent, int nRecent, float r, int* token);
    [DllImport(Lib)] public static extern int llmdot_hip_sample_noalloc(nint ctx, float* logitsDev, int n, Sampling* opt, int* recentDev, int nRecent, float r, int* tokenDev);

    // ---- device memory and timing hooks ------------------------------------------
    [DllImport(Lib)] public static extern int llmdot_hip_device_alloc(nint ctx, nuint nbytes, void** dptr);
    [DllImport(Lib)] public static extern int llmdot_hip_device_free(nint ctx, void* dptr);
    [DllImport(Lib)] public static extern int llmdot_hip_memcpy_h2d(nint ctx, void* dst, void* src, nuint nbytes);
    [DllImport(Lib)] public static extern int llmdot_hip_memcpy_d2h(nint ctx, void* dst, void* src, nuint nbytes);
    [DllImport(Lib)] public static extern int llmdot_hip_synchronize(nint ctx);
    [DllImport(Lib)] public static extern int llmdot_hip_gemv_device(nint ctx, uint ggmlType, void* wDev, float* xDev, float* yDev, int rows, int cols);
    [DllImport(Lib)] public static extern int llmdot_hip_time_gemv(nint ctx, uint ggmlType, void** wDevs, int nWeights, float* xDev, float* yDev, int rows, int cols, int iters, float* ms);
    [DllImport(Lib)] public static extern int llmdot_hip_stream_bench(nint ctx, nuint nbytes, int mode, int iters, float* ms);

    // ---- model level: the device-resident decode step ---------------------------
    [DllImport(Lib)] public static extern int llmdot_hip_model_create(nint ctx, ModelDesc* desc, nint* model);
    [DllImport(Lib)] public static extern int llmdot_hip_model_destroy(nint model);
    [DllImport(Lib)] public static extern int llmdot_hip_model_reset(nint model);
    [DllImport(Lib)] public static extern int llmdot_hip_decode_step(nint model, int token, int position, float* logitsOrNull, int* argmaxOrNull);
    [DllImport(Lib)] public static extern int llmdot_hip_prefill(nint model, int* tokens, int n, int pos0, float* logitsOrNull, int* argmaxOrNull);
    [DllImport(Lib)] public static extern int llmdot_hip_generate(nint model, int* prompt, int nPrompt, int maxTokens, int eos, int* tokensOut, int* nOut, float* logitsOut);
    [DllImport(Lib)] public static extern int llmdot_hip_generate_sampled(nint model, int* prompt, int nPrompt, int maxTokens, int eos, Sampling* opt, float* draws, int* tokensOut, int* nOut, float* logitsOut);
    [DllImport(Lib)] public static extern int llmdot_hip_generate_begin(nint model, int* prompt, int nPrompt, int maxTokens, int eos, Sampling* optOrNull, float* drawsOrNull);
    [DllImport(Lib)] public static extern int llmdot_hip_generate_next(nint model, int maxK, int* tokensOut, int* nOut, int* done, float* logitsOutOrNull);
    [DllImport(Lib)] public static extern int llmdot_hip_kv_read(nint model, int layer, int position, float* k, float* v);
    [DllImport(Lib)] public static extern int llmdot_hip_model_time_prefill(nint model, int* tokens, int n, int pos0, float* ms);
    [DllImport(Lib)] public static extern int llmdot_hip_model_time_decode(nint model, int firstToken, int position, int steps, int perKernel, StepTiming* timing);
    [DllImport(Lib)] public static extern int llmdot_hip_model_step_bytes(nint model, int position, double* bytes);
    [DllImport(Lib)] public static extern int llmdot_hip_model_kv_fill_random(nint model, int n, ulong seed);

    // ---- GGUF tooling (host only) -----------------------------------------------
    [DllImport(Lib)] public static extern int llmdot_hip_quantize(uint ggmlType, float* src, long rows, long cols, void* dst);
    [DllImport(Lib)] public static extern int llmdot_hip_synth_weights(uint ggmlType, long rows, long cols, ulong seed, float sigma, void* dst, int threads);

    /// <summary>The library's message for the last failure on this thread.</summary>
    public static string LastError() => Marshal.PtrToStringUTF8(llmdot_hip_last_error()) ?? string.Empty;

    /// <summary>Throws the exception the reference raises for the condition a status code reports.</summary>
    public static void Check(int rc)
    {
        if (rc == Ok) return;
        var msg = LastError();
        throw rc switch
        {
            EInvalid => new ArgumentException(msg),
            EUnsupported => new NotSupportedException(msg),
            ENotFound => new KeyNotFoundException(msg),
            ERange => new ArgumentOutOfRangeException(null, msg),
            ENoMem => new OutOfMemoryException(msg),
            _ => new InvalidOperationException($"HIP device error: {msg}"),
        };
    }

    /// <summary>NUL-terminated UTF-8 copy of a managed string (null stays null).</summary>
    public static byte[]? Utf8(string? s) => s is null ? null : System.Text.Encoding.UTF8.GetBytes(s + "\0");

    /// <summary>True when the library loads and reports at least one device.</summary>
    public static bool TryDeviceCount(out int count)
    {
        count = 0;
        try
        {
            if (!NativeLibrary.TryLoad("libllmdot_hip.so", typeof(HipNative).Assembly, null, out _) &&
                !NativeLibrary.TryLoad("llmdot_hip", typeof(HipNative).Assembly, null, out _))
                return false;
            int n;
            if (llmdot_hip_device_count(&n) != Ok) return false;
            count = n;
            return n > 0;
        }
        catch (DllNotFoundException)
        {
            return false;
        }
        catch (EntryPointNotFoundException)
        {
            return false;
        }
    }
}
