"""Model integrations (mirror of src/refinekv/integrations/)."""
