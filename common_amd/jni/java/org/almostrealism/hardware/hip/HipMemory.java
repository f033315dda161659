/*
 * One device allocation of a HipMemoryProvider: a HIP device pointer and its size in bytes.
 * The RAM subclass the reference's providers hand out (base/hardware/src/main/java/org/
 * almostrealism/hardware/mem/RAM.java; the Metal counterpart is metal/MetalMemory.java).
 *
 * Not compiled in this repository (no JDK in the build image).
 */
package org.almostrealism.hardware.hip;

import org.almostrealism.hardware.mem.RAM;

public class HipMemory extends RAM {
	private final HipMemoryProvider provider;
	private final long pointer;
	private final long bytes;

	HipMemory(HipMemoryProvider provider, long pointer, long bytes) {
		this.provider = provider;
		this.pointer = pointer;
		this.bytes = bytes;
	}

	@Override
	public HipMemoryProvider getProvider() { return provider; }

	/** The device address (what the C-ABI takes as a pointer). */
	@Override
	public long getContentPointer() { return pointer; }

	/** Size in bytes: elements x the provider's number size. */
	@Override
	public long getSize() { return bytes; }
}
