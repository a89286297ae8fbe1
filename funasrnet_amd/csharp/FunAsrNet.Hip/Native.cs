using System.Runtime.InteropServices;

namespace FunAsrNet.Hip;

/// <summary>P/Invoke surface of libfunasr_hip.so (include/funasr_hip.h). The
/// library is found by name ("funasr_hip"), or at the absolute path in
/// FUNASRNET_HIP_LIBRARY, as src/FunAsrNet.Vulkan/Vendor/Vk.cs:13-47 resolves
/// vulkan-1.</summary>
internal static unsafe partial class Native
{
    private const string Lib = "funasr_hip";

    static Native()
    {
        NativeLibrary.SetDllImportResolver(typeof(Native).Assembly, (name, assembly, path) =>
        {
            if (name != Lib)
            {
                return IntPtr.Zero;
            }
            string? overridePath = Environment.GetEnvironmentVariable("FUNASRNET_HIP_LIBRARY");
            return overridePath is { Length: > 0 } ? NativeLibrary.Load(overridePath) : IntPtr.Zero;
        });
    }

    internal const int Ok = 0, Declined = 1, ErrorArgument = -1, ErrorDevice = -2, ErrorDisposed = -3, ErrorState = -4;

    [StructLayout(LayoutKind.Sequential)]
    internal struct DecoderConfig
    {
        public int Width, Heads, KvHeads, HeadSize, Layers, Ffn, Vocab;
        public float Eps, RopeBase;
        public int Capacity;
    }

    [StructLayout(LayoutKind.Sequential)]
    internal struct Q8Host
    {
        public sbyte* Quantized;
        public float* Scales;
        public int Rows, Cols;
        public byte* Blocks;
    }

    [StructLayout(LayoutKind.Sequential)]
    internal struct LayerHost
    {
        public Q8Host Wq, Wk, Wv, Wo, Gate, Up, Down;
        public float* AttnNorm, QNorm, KNorm, FfnNorm;
    }

    /// <summary>fah_call_stats: one seam entry point's counters.</summary>
    [StructLayout(LayoutKind.Sequential)]
    internal struct CallStats
    {
        public long Calls, Declined, Operations, UploadedBytes, DownloadedBytes;
        public double DeviceMilliseconds, TotalMilliseconds;
    }

    /// <summary>FAH_CALL_* order of fah_context_statistics.</summary>
    internal static readonly string[] CallKinds =
        ["quantizedLinear", "quantizedLinearNoAlloc", "linearMany", "linear", "reluProjection", "attention"];

    [LibraryImport(Lib)] internal static partial int fah_abi_version();
    [LibraryImport(Lib)] internal static partial int fah_context_statistics(IntPtr context, CallStats* stats, int kinds);
    [LibraryImport(Lib)] internal static partial int fah_context_reset_statistics(IntPtr context);
    [LibraryImport(Lib)] internal static partial IntPtr fah_last_error();
    [LibraryImport(Lib)] internal static partial int fah_device_count();
    [LibraryImport(Lib)] internal static partial int fah_context_create(int device, out IntPtr context);
    [LibraryImport(Lib)] internal static partial int fah_context_destroy(IntPtr context);
    [LibraryImport(Lib)] internal static partial IntPtr fah_context_name(IntPtr context);
    [LibraryImport(Lib)] internal static partial int fah_context_set_minimum_operations(IntPtr context, long operations);

    [LibraryImport(Lib)] internal static partial int fah_weight_q8_upload(IntPtr context, sbyte* quantized, float* scales, int rows, int cols, out IntPtr weight);
    [LibraryImport(Lib)] internal static partial int fah_weight_f32_upload(IntPtr context, float* values, int rows, int cols, out IntPtr weight);
    [LibraryImport(Lib)] internal static partial int fah_weight_release(IntPtr weight);

    [LibraryImport(Lib)] internal static partial int fah_quantized_linear(IntPtr context, float* input, int frames, IntPtr weight, float* bias, float* output);
    [LibraryImport(Lib)] internal static partial int fah_linear(IntPtr context, float* input, int frames, IntPtr weight, float* bias, float* output);
    [LibraryImport(Lib)] internal static partial int fah_linear_many(IntPtr context, float* input, int frames, IntPtr* weights, int count, float** outputs);
    [LibraryImport(Lib)] internal static partial int fah_relu_projection(IntPtr context, float* input, int frames, IntPtr first, float* firstBias, IntPtr second, float* secondBias, float* output);
    [LibraryImport(Lib)] internal static partial int fah_attention(IntPtr context, float* query, float* key, float* value, int frames, int width, int heads, float* output);

    [LibraryImport(Lib)] internal static partial int fah_decoder_create(IntPtr context, DecoderConfig* config, LayerHost* layers, Q8Host* tokenEmbd, Q8Host* output, float* outputNorm, out IntPtr decoder);
    [LibraryImport(Lib)] internal static partial int fah_decoder_destroy(IntPtr decoder);
    [LibraryImport(Lib)] internal static partial int fah_decoder_set_position(IntPtr decoder, int position);
    [LibraryImport(Lib)] internal static partial int fah_decoder_position(IntPtr decoder, out int position);
    [LibraryImport(Lib)] internal static partial int fah_decoder_decode(IntPtr decoder, float* embeddings, int frames, float* logits);
    [LibraryImport(Lib)] internal static partial int fah_decoder_embed(IntPtr decoder, int* tokens, int count, float* output);
    [LibraryImport(Lib)] internal static partial int fah_decoder_greedy(IntPtr decoder, out int token);
    [LibraryImport(Lib)] internal static partial int fah_decoder_generate(IntPtr decoder, int steps, int* tokens);
    [LibraryImport(Lib)] internal static partial int fah_decoder_create_session(IntPtr parent, int capacity, out IntPtr session);

    [LibraryImport(Lib)] internal static partial int fah_batcher_create(IntPtr parent, int maxPositions, int windowMicroseconds, out IntPtr batcher);
    [LibraryImport(Lib)] internal static partial int fah_batcher_destroy(IntPtr batcher);
    [LibraryImport(Lib)] internal static partial int fah_batcher_join(IntPtr batcher, IntPtr session);
    [LibraryImport(Lib)] internal static partial int fah_batcher_leave(IntPtr batcher, IntPtr session);
    [LibraryImport(Lib)] internal static partial int fah_batcher_step(IntPtr batcher, IntPtr session, out int token);

    /// <summary>0 = done, 1 = declined (the Try* method returns false with the
    /// output untouched), negative = error, thrown with the library's message
    /// as the reference throws it (VulkanQuantizedBackend.cs:49-56, Vk.cs:57-61).</summary>
    internal static bool Check(int rc)
    {
        if (rc == Ok)
        {
            return true;
        }
        if (rc > 0)
        {
            return false;
        }
        string message = Marshal.PtrToStringUTF8(fah_last_error()) ?? "funasr_hip error";
        throw rc switch
        {
            ErrorArgument => new ArgumentException(message),
            ErrorDisposed => new ObjectDisposedException(message),
            _ => new InvalidOperationException(message),
        };
    }
}
