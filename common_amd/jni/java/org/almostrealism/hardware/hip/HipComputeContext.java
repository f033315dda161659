/*
 * ComputeContext of a HipDataContext (base/code/src/main/java/io/almostrealism/code/
 * ComputeContext.java:59-150, through AbstractComputeContext).
 *
 * isCPU() is false; copy() between two HipMemory regions is one device-to-device copy on the GPU's
 * stream (element offsets x 4 bytes, as in HipMemoryProvider), any other pair goes through
 * AbstractComputeContext's host path.  deliver(Scope) is refused: this backend runs the Qwen3
 * decode / prefill step as hand-written kernels behind the C-ABI (HipQwen3) and does not compile
 * generated scopes, which stay with the CPU contexts.
 *
 * Not compiled in this repository (no JDK in the build image).
 */
package org.almostrealism.hardware.hip;

import io.almostrealism.code.InstructionSet;
import io.almostrealism.lang.LanguageOperations;
import io.almostrealism.scope.Scope;
import io.almostrealism.streams.Semaphore;
import org.almostrealism.hardware.MemoryData;
import org.almostrealism.hardware.ctx.AbstractComputeContext;

public class HipComputeContext extends AbstractComputeContext<HipDataContext> {
	HipComputeContext(HipDataContext dc) {
		super(dc);
	}

	@Override
	public LanguageOperations getLanguage() {
		throw new UnsupportedOperationException("HIP context has no code generator (hand-written kernels only)");
	}

	@Override
	public InstructionSet deliver(Scope scope) {
		throw new UnsupportedOperationException("HIP context runs the Qwen3 decode / prefill step only; scope "
				+ scope.getName() + " belongs on a CPU compute context");
	}

	@Override
	public boolean isCPU() { return false; }

	@Override
	public Semaphore copy(MemoryData source, MemoryData destination, Semaphore dependsOn) {
		if (source.getMem() instanceof HipMemory src && destination.getMem() instanceof HipMemory dst) {
			if (dependsOn != null) dependsOn.waitFor();
			long n = src.getProvider().getNumberSize();
			HIP.copy(getDataContext().getHandle(), dst.getContentPointer() + destination.getOffset() * n,
					src.getContentPointer() + source.getOffset() * n, source.getMemLength() * n);
			return null;  /* ordered on the stream: a later host read waits for it */
		}
		return super.copy(source, destination, dependsOn);
	}

	/** Waits for every copy and kernel enqueued on the GPU's stream. */
	public void synchronize() { HIP.synchronize(getDataContext().getHandle()); }

	@Override
	public void destroy() { }
}
