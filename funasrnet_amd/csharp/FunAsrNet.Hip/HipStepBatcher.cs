namespace FunAsrNet.Hip;

/// <summary>Cross-context step batching (fah_batcher_*) for the worker threads of a
/// BoundedInferencePool (BoundedInferencePool.cs:22-230) over the N FunAsr
/// contexts of SpeechRuntime (SpeechRuntime.cs:16-23): each worker's decoder
/// steps through <see cref="Step"/>, and the steps the workers request at the
/// same time run as one lock-step batch over the shared device weights.</summary>
public sealed class HipStepBatcher : IDisposable
{
    private readonly object _gate = new();
    private IntPtr _batcher;
    private int _users;   // decoders stepping through this batcher

    /// <param name="maxPositions">Position bound of the batched steps (the first
    /// decoder's capacity, at most 15360); decoders past it step on their own.</param>
    internal HipStepBatcher(IntPtr parentDecoder, int maxPositions, int windowMicroseconds = 2000)
    {
        Native.Check(Native.fah_batcher_create(parentDecoder, maxPositions, windowMicroseconds, out _batcher));
        MaxPositions = maxPositions;
    }

    internal int MaxPositions { get; }

    private IntPtr Live
    {
        get
        {
            ObjectDisposedException.ThrowIf(_batcher == IntPtr.Zero, this);
            return _batcher;
        }
    }

    internal void AddUser()
    {
        lock (_gate)
        {
            ObjectDisposedException.ThrowIf(_batcher == IntPtr.Zero, this);
            _users++;
        }
    }

    /// <summary>The last decoder to let go destroys the native batcher (its
    /// weights and context stay alive in the library until then).</summary>
    internal void ReleaseUser()
    {
        lock (_gate)
        {
            if (--_users == 0)
            {
                Dispose();
            }
        }
    }

    /// <summary>Registers a decoder whose steps the collecting thread waits for.</summary>
    internal void Join(HipDecoderStep step) => Native.Check(Native.fah_batcher_join(Live, step.Handle));

    internal void Leave(HipDecoderStep step) => Native.Check(Native.fah_batcher_leave(Live, step.Handle));

    /// <summary>One greedy step of <paramref name="step"/>'s decoder, batched with
    /// the other workers' concurrent steps; blocks until it has run. An error of
    /// this decoder's step (its capacity reached) is thrown here alone.</summary>
    internal int Step(HipDecoderStep step)
    {
        Native.Check(Native.fah_batcher_step(Live, step.Handle, out int token));
        return token;
    }

    public void Dispose()
    {
        lock (_gate)
        {
            if (_batcher != IntPtr.Zero)
            {
                Native.Check(Native.fah_batcher_destroy(_batcher));
                _batcher = IntPtr.Zero;
            }
        }
    }
}
